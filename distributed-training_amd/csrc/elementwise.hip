// Elementwise and reduction kernels behind dtrain's generic Tensor ops
// (dtrain/autograd.py:29-148): strided copies (reshape/transpose of
// non-contiguous views), broadcasting add/sub/mul, scaling by a host or device
// scalar, GELU and ReLU forward/backward, general axis sums (_unbroadcast,
// Tensor.sum) and the deterministic two-stage column sum used for bias
// gradients.
//
// The big-array kernels (GELU, binary same-shape, column sums) are HBM-bound:
// 16-byte vector access when aligned, grid-stride loops, no atomics.
#include <cmath>

#include "colreduce.h"
#include "common.h"
#include "gelu.h"

namespace dtmi {

constexpr int kMaxDims = 8;

struct Shape8 {
  int64_t shape[kMaxDims];
  int64_t s0[kMaxDims];  // strides (elements) of operand 0
  int64_t s1[kMaxDims];  // strides of operand 1
  int64_t s2[kMaxDims];  // strides of operand 2 (output)
  int ndim;
};

__device__ __forceinline__ void offsets3(const Shape8& sh, int64_t lin, int64_t& o0, int64_t& o1, int64_t& o2) {
  o0 = o1 = o2 = 0;
  for (int d = sh.ndim - 1; d >= 0; --d) {
    int64_t s = sh.shape[d];
    int64_t i = lin % s;
    lin /= s;
    o0 += i * sh.s0[d];
    o1 += i * sh.s1[d];
    o2 += i * sh.s2[d];
  }
}

static int grid_1d(int64_t n, int per_thread = 4) {
  int64_t b = cdiv(n, 256LL * per_thread);
  if (b < 1) b = 1;
  return (int)(b < 4096 ? b : 4096);
}

// ------------------------------------------------------------ copies
template <typename T>
__global__ void copy_strided_kernel(T* __restrict__ dst, const T* __restrict__ src, Shape8 sh, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t lin = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; lin < n; lin += stride) {
    int64_t os, od, unused;
    offsets3(sh, lin, os, unused, od);
    dst[od] = src[os];
  }
}

// ------------------------------------------------------------ binary
enum BinOp { kAdd = 0, kSub = 1, kMul = 2 };

template <typename T, int OP>
__device__ __forceinline__ T binop(T a, T b) {
  if (OP == kAdd) return a + b;
  if (OP == kSub) return a - b;
  return a * b;
}

template <typename T, int OP>
__global__ void binary_strided_kernel(T* __restrict__ out, const T* __restrict__ a, const T* __restrict__ b, Shape8 sh,
                                      int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t lin = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; lin < n; lin += stride) {
    int64_t oa, ob, oo;
    offsets3(sh, lin, oa, ob, oo);
    out[oo] = binop<T, OP>(a[oa], b[ob]);
  }
}

template <typename T, int OP>
__global__ void binary_same_kernel(T* __restrict__ out, const T* __restrict__ a, const T* __restrict__ b, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (aligned(out, 16) && aligned(a, 16) && aligned(b, 16)) {
    constexpr int N = 16 / sizeof(T);
    const int64_t nv = n / N;
    for (int64_t i = tid; i < nv; i += stride) {
      T va[N], vb[N];
      *reinterpret_cast<uint4*>(va) = reinterpret_cast<const uint4*>(a)[i];
      *reinterpret_cast<uint4*>(vb) = reinterpret_cast<const uint4*>(b)[i];
#pragma unroll
      for (int e = 0; e < N; ++e) va[e] = binop<T, OP>(va[e], vb[e]);
      reinterpret_cast<uint4*>(out)[i] = *reinterpret_cast<uint4*>(va);
    }
    for (int64_t k = nv * N + tid; k < n; k += stride) out[k] = binop<T, OP>(a[k], b[k]);
  } else {
    for (int64_t k = tid; k < n; k += stride) out[k] = binop<T, OP>(a[k], b[k]);
  }
}

// out[r, c] = a[r, c] (op) b[c]  (row-broadcast of a bias vector)
template <typename T, int OP>
__global__ void binary_rowbcast_kernel(T* __restrict__ out, const T* __restrict__ a, const T* __restrict__ b,
                                       int64_t rows, int64_t cols) {
  const int64_t n = rows * cols;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; k < n; k += stride)
    out[k] = binop<T, OP>(a[k], b[k % cols]);
}

// ------------------------------------------------------------ scale
template <typename T>
__global__ void scale_kernel(T* __restrict__ out, const T* __restrict__ x, int64_t n, T alpha,
                             const T* __restrict__ alpha_dev) {
  const T s = alpha_dev ? *alpha_dev : alpha;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; k < n; k += stride) out[k] = x[k] * s;
}

// ------------------------------------------------------------ GELU / ReLU
// tanh-GELU exactly as dtrain/autograd.py:133-144 writes it:
//   c = sqrt(2/pi) (rounded to T); u = c * (x + 0.044715 * x^3); t = tanh(u)
//   y = 0.5 * x * (1 + t)
//   dx = g * (0.5 * (1 + t) + 0.5 * x * (1 - t*t) * (c * (1 + 3*0.044715 * x^2)))
template <typename T, bool BWD>
__global__ void __launch_bounds__(256) gelu_kernel(T* __restrict__ out, const T* __restrict__ x,
                                                    const T* __restrict__ g, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  bool vec = aligned(out, 16) && aligned(x, 16) && (!BWD || aligned(g, 16));
  if (vec) {
    constexpr int N = 16 / sizeof(T);
    const int64_t nv = n / N;
    for (int64_t i = tid; i < nv; i += stride) {
      T vx[N], vg[N];
      *reinterpret_cast<uint4*>(vx) = reinterpret_cast<const uint4*>(x)[i];
      if (BWD) *reinterpret_cast<uint4*>(vg) = reinterpret_cast<const uint4*>(g)[i];
#pragma unroll
      for (int e = 0; e < N; ++e) vx[e] = BWD ? gelu_b<T>(vx[e], vg[e]) : gelu_f<T>(vx[e]);
      reinterpret_cast<uint4*>(out)[i] = *reinterpret_cast<uint4*>(vx);
    }
    for (int64_t k = nv * N + tid; k < n; k += stride) out[k] = BWD ? gelu_b<T>(x[k], g[k]) : gelu_f<T>(x[k]);
  } else {
    for (int64_t k = tid; k < n; k += stride) out[k] = BWD ? gelu_b<T>(x[k], g[k]) : gelu_f<T>(x[k]);
  }
}

// relu: y = x * (x > 0); dx = g * (x > 0)   (dtrain/autograd.py:146-148)
template <typename T, bool BWD>
__global__ void relu_kernel(T* __restrict__ out, const T* __restrict__ x, const T* __restrict__ g, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; k < n; k += stride) {
    T m = x[k] > T(0) ? T(1) : T(0);
    out[k] = BWD ? g[k] * m : x[k] * m;
  }
}

// ------------------------------------------------------------ reductions
// General sum of a strided input over the axes whose output stride is 0:
// output element o (contiguous, `nout` of them) sums its `nred` inputs in
// row-major order of the reduced axes. One thread per output.
struct ReduceDesc {
  int64_t out_shape[kMaxDims];  // kept axes (size 1 for reduced ones)
  int64_t in_strides_kept[kMaxDims];
  int64_t red_shape[kMaxDims];  // reduced axes (size 1 for kept ones)
  int64_t in_strides_red[kMaxDims];
  int ndim;
};

template <typename T>
__global__ void reduce_axes_kernel(T* __restrict__ out, const T* __restrict__ x, ReduceDesc d, int64_t nout,
                                   int64_t nred) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; o < nout; o += stride) {
    int64_t base = 0, lin = o;
    for (int k = d.ndim - 1; k >= 0; --k) {
      int64_t s = d.out_shape[k];
      base += (lin % s) * d.in_strides_kept[k];
      lin /= s;
    }
    T acc = T(0);
    for (int64_t r = 0; r < nred; ++r) {
      int64_t off = 0, l2 = r;
      for (int k = d.ndim - 1; k >= 0; --k) {
        int64_t s = d.red_shape[k];
        off += (l2 % s) * d.in_strides_red[k];
        l2 /= s;
      }
      acc = acc + x[base + off];
    }
    out[o] = acc;
  }
}

// Sum over leading axes of a contiguous array, viewed as [nred, nout]:
// out[o] = sum_r x[r * nout + o] with r ascending, the order of
// reduce_axes_kernel for this case (the same bits), in 16-byte vectors with
// eight rows of loads in flight per thread.
template <typename T>
__global__ void __launch_bounds__(256) reduce_lead_kernel(T* __restrict__ out, const T* __restrict__ x, int64_t nout,
                                                           int64_t nred) {
  constexpr int N = 16 / sizeof(T);
  typedef T vt __attribute__((ext_vector_type(N)));
  const int64_t nv = nout / N;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nv; i += stride) {
    const T* p = x + i * N;
    vt acc = (vt)(T(0));
    int64_t r = 0;
    for (; r + 8 <= nred; r += 8) {
      vt v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = *reinterpret_cast<const vt*>(p + (r + u) * nout);
#pragma unroll
      for (int u = 0; u < 8; ++u) acc = acc + v[u];
    }
    for (; r < nred; ++r) acc = acc + *reinterpret_cast<const vt*>(p + r * nout);
    *reinterpret_cast<vt*>(out + i * N) = acc;
  }
}

// Column sums of a [rows, cols] row-major matrix, deterministic two-stage:
// stage 1 block (bx, by) sums rows [by*RB, (by+1)*RB) of columns
// [bx*256*V, ...) into part[by][col]; stage 2 sums the parts of each column in
// increasing `by` order. Coalesced: consecutive threads read consecutive columns.
constexpr int kColRows = 128;

template <typename T>
__global__ void __launch_bounds__(256) colsum_stage1_kernel(T* __restrict__ part, const T* __restrict__ x,
                                                             int64_t rows, int64_t cols) {
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= cols) return;
  const int64_t r0 = (int64_t)blockIdx.y * kColRows;
  const int64_t r1 = r0 + kColRows < rows ? r0 + kColRows : rows;
  T acc = T(0);
  int64_t r = r0;
  for (; r + 8 <= r1; r += 8) {
    T v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = x[(r + u) * cols + c];
#pragma unroll
    for (int u = 0; u < 8; ++u) acc = acc + v[u];
  }
  for (; r < r1; ++r) acc = acc + x[r * cols + c];
  part[(int64_t)blockIdx.y * cols + c] = acc;
}

template <typename T>
static int fill_shape8(Shape8& sh, int ndim, const int64_t* shape, const int64_t* st0, const int64_t* st1,
                       const int64_t* st2, int64_t* n_out) {
  DTMI_CHECK(ndim >= 0 && ndim <= kMaxDims, "at most %d dimensions (got %d)", kMaxDims, ndim);
  int64_t n = 1;
  sh.ndim = ndim;
  for (int d = 0; d < kMaxDims; ++d) {
    sh.shape[d] = 1;
    sh.s0[d] = sh.s1[d] = sh.s2[d] = 0;
  }
  // contiguous strides for NULL stride arrays
  int64_t acc = 1;
  for (int d = ndim - 1; d >= 0; --d) {
    DTMI_CHECK(shape[d] >= 0, "negative dimension");
    sh.shape[d] = shape[d];
    sh.s0[d] = st0 ? st0[d] : acc;
    sh.s1[d] = st1 ? st1[d] : acc;
    sh.s2[d] = st2 ? st2[d] : acc;
    acc *= shape[d];
  }
  for (int d = 0; d < ndim; ++d) n *= shape[d];
  *n_out = n;
  return DTMI_OK;
}

}  // namespace dtmi

using namespace dtmi;

DTMI_EXPORT int dtmi_copy_strided(int dtype, void* dst, const int64_t* dst_strides, const void* src,
                                  const int64_t* src_strides, int ndim, const int64_t* shape) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_DTYPE_OK(dtype);
  Shape8 sh;
  int64_t n = 0;
  int rc = dtype == DTMI_F32 ? fill_shape8<float>(sh, ndim, shape, src_strides, nullptr, dst_strides, &n)
                             : fill_shape8<double>(sh, ndim, shape, src_strides, nullptr, dst_strides, &n);
  if (rc) return rc;
  if (n == 0) return DTMI_OK;
  DTMI_CHECK(dst && src, "dtmi_copy_strided: NULL pointer");
  TimedLaunch tl(DTMI_FAM_OTHER, 2.0 * (double)n * (dtype == DTMI_F32 ? 4 : 8));
  if (dtype == DTMI_F32)
    copy_strided_kernel<float><<<grid_1d(n), 256, 0, stream()>>>((float*)dst, (const float*)src, sh, n);
  else
    copy_strided_kernel<double><<<grid_1d(n), 256, 0, stream()>>>((double*)dst, (const double*)src, sh, n);
  LAUNCH_CHECK("copy_strided_kernel");
  return DTMI_OK;
  DTMI_BODY_END
}

template <typename T, int OP>
static void launch_binary(void* out, const void* a, const int64_t* sa, const void* b, const int64_t* sb, int ndim,
                          const int64_t* shape, const Shape8& sh, int64_t n) {
  // fast paths: same-shape contiguous, or [rows, cols] (op) [cols] bias
  bool a_contig = true, b_contig = true;
  {
    int64_t acc = 1;
    for (int d = ndim - 1; d >= 0; --d) {
      if (shape[d] != 1 && sa && sa[d] != acc) a_contig = false;
      if (shape[d] != 1 && sb && sb[d] != acc) b_contig = false;
      acc *= shape[d];
    }
  }
  if (a_contig && b_contig) {
    binary_same_kernel<T, OP><<<grid_1d(n), 256, 0, stream()>>>((T*)out, (const T*)a, (const T*)b, n);
    return;
  }
  if (a_contig && ndim >= 1 && sb) {
    bool rowb = sb[ndim - 1] == 1 || shape[ndim - 1] == 1;
    for (int d = 0; d < ndim - 1; ++d)
      if (sb[d] != 0 && shape[d] != 1) rowb = false;
    if (rowb && shape[ndim - 1] > 0 && (sb[ndim - 1] == 1)) {
      int64_t cols = shape[ndim - 1];
      binary_rowbcast_kernel<T, OP><<<grid_1d(n), 256, 0, stream()>>>((T*)out, (const T*)a, (const T*)b, n / cols,
                                                                       cols);
      return;
    }
  }
  binary_strided_kernel<T, OP><<<grid_1d(n), 256, 0, stream()>>>((T*)out, (const T*)a, (const T*)b, sh, n);
}

// out (contiguous, `shape`) = a (op) b with element strides sa / sb (0 on
// broadcast axes; NULL = contiguous).
DTMI_EXPORT int dtmi_binary(int dtype, int op, void* out, const void* a, const int64_t* a_strides, const void* b,
                            const int64_t* b_strides, int ndim, const int64_t* shape) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_DTYPE_OK(dtype);
  DTMI_CHECK(op >= 0 && op <= 2, "dtmi_binary: bad op %d", op);
  Shape8 sh;
  int64_t n = 0;
  int rc = fill_shape8<float>(sh, ndim, shape, a_strides, b_strides, nullptr, &n);
  if (rc) return rc;
  if (n == 0) return DTMI_OK;
  DTMI_CHECK(out && a && b, "dtmi_binary: NULL pointer");
  TimedLaunch tl(DTMI_FAM_OTHER, 3.0 * (double)n * (dtype == DTMI_F32 ? 4 : 8));
#define BIN_CASE(T, OPV) launch_binary<T, OPV>(out, a, a_strides, b, b_strides, ndim, shape, sh, n)
  if (dtype == DTMI_F32) {
    if (op == kAdd) BIN_CASE(float, kAdd);
    else if (op == kSub) BIN_CASE(float, kSub);
    else BIN_CASE(float, kMul);
  } else {
    if (op == kAdd) BIN_CASE(double, kAdd);
    else if (op == kSub) BIN_CASE(double, kSub);
    else BIN_CASE(double, kMul);
  }
#undef BIN_CASE
  LAUNCH_CHECK("binary kernel");
  return DTMI_OK;
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_scale(int dtype, void* out, const void* x, int64_t n, double alpha, const void* alpha_dev) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_DTYPE_OK(dtype);
  DTMI_CHECK(n >= 0, "dtmi_scale: negative size");
  if (n == 0) return DTMI_OK;
  DTMI_CHECK(out && x, "dtmi_scale: NULL pointer");
  TimedLaunch tl(DTMI_FAM_OTHER, 2.0 * (double)n * (dtype == DTMI_F32 ? 4 : 8));
  if (dtype == DTMI_F32)
    scale_kernel<float><<<grid_1d(n), 256, 0, stream()>>>((float*)out, (const float*)x, n, (float)alpha,
                                                          (const float*)alpha_dev);
  else
    scale_kernel<double><<<grid_1d(n), 256, 0, stream()>>>((double*)out, (const double*)x, n, alpha,
                                                           (const double*)alpha_dev);
  LAUNCH_CHECK("scale_kernel");
  return DTMI_OK;
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_gelu_fwd(int dtype, void* y, const void* x, int64_t n) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_DTYPE_OK(dtype);
  DTMI_CHECK(n >= 0, "dtmi_gelu_fwd: negative size");
  if (n == 0) return DTMI_OK;
  DTMI_CHECK(y && x, "dtmi_gelu_fwd: NULL pointer");
  TimedLaunch tl(DTMI_FAM_OTHER, 2.0 * (double)n * (dtype == DTMI_F32 ? 4 : 8));
  if (dtype == DTMI_F32)
    gelu_kernel<float, false><<<grid_1d(n, 8), 256, 0, stream()>>>((float*)y, (const float*)x, nullptr, n);
  else
    gelu_kernel<double, false><<<grid_1d(n, 4), 256, 0, stream()>>>((double*)y, (const double*)x, nullptr, n);
  LAUNCH_CHECK("gelu_kernel");
  return DTMI_OK;
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_gelu_bwd(int dtype, void* dx, const void* x, const void* dy, int64_t n) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_DTYPE_OK(dtype);
  DTMI_CHECK(n >= 0, "dtmi_gelu_bwd: negative size");
  if (n == 0) return DTMI_OK;
  DTMI_CHECK(dx && x && dy, "dtmi_gelu_bwd: NULL pointer");
  TimedLaunch tl(DTMI_FAM_GELU_BWD, 3.0 * (double)n * (dtype == DTMI_F32 ? 4 : 8));
  if (dtype == DTMI_F32)
    gelu_kernel<float, true><<<grid_1d(n, 8), 256, 0, stream()>>>((float*)dx, (const float*)x, (const float*)dy, n);
  else
    gelu_kernel<double, true><<<grid_1d(n, 4), 256, 0, stream()>>>((double*)dx, (const double*)x,
                                                                   (const double*)dy, n);
  LAUNCH_CHECK("gelu_kernel");
  return DTMI_OK;
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_relu_fwd(int dtype, void* y, const void* x, int64_t n) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_DTYPE_OK(dtype);
  if (n <= 0) return n == 0 ? DTMI_OK : dtmi::fail(DTMI_ERR_INVALID, "dtmi_relu_fwd: negative size");
  DTMI_CHECK(y && x, "dtmi_relu_fwd: NULL pointer");
  if (dtype == DTMI_F32)
    relu_kernel<float, false><<<grid_1d(n), 256, 0, stream()>>>((float*)y, (const float*)x, nullptr, n);
  else
    relu_kernel<double, false><<<grid_1d(n), 256, 0, stream()>>>((double*)y, (const double*)x, nullptr, n);
  LAUNCH_CHECK("relu_kernel");
  return DTMI_OK;
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_relu_bwd(int dtype, void* dx, const void* x, const void* dy, int64_t n) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_DTYPE_OK(dtype);
  if (n <= 0) return n == 0 ? DTMI_OK : dtmi::fail(DTMI_ERR_INVALID, "dtmi_relu_bwd: negative size");
  DTMI_CHECK(dx && x && dy, "dtmi_relu_bwd: NULL pointer");
  if (dtype == DTMI_F32)
    relu_kernel<float, true><<<grid_1d(n), 256, 0, stream()>>>((float*)dx, (const float*)x, (const float*)dy, n);
  else
    relu_kernel<double, true><<<grid_1d(n), 256, 0, stream()>>>((double*)dx, (const double*)x, (const double*)dy, n);
  LAUNCH_CHECK("relu_kernel");
  return DTMI_OK;
  DTMI_BODY_END
}

// Sum of x (shape `shape`, element strides `strides`, NULL = contiguous) over
// the axes with reduce_mask[d] != 0, into contiguous `out` holding the kept
// axes in order.
DTMI_EXPORT int dtmi_reduce_sum(int dtype, void* out, const void* x, const int64_t* strides, int ndim,
                                const int64_t* shape, const int* reduce_mask) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_DTYPE_OK(dtype);
  DTMI_CHECK(ndim >= 0 && ndim <= kMaxDims, "dtmi_reduce_sum: at most %d dims", kMaxDims);
  DTMI_CHECK(ndim == 0 || (shape && reduce_mask), "dtmi_reduce_sum: NULL shape/mask");
  ReduceDesc d;
  d.ndim = ndim;
  int64_t nout = 1, nred = 1, acc = 1;
  int64_t cstr[kMaxDims];
  for (int k = ndim - 1; k >= 0; --k) {
    cstr[k] = acc;
    acc *= shape[k];
  }
  for (int k = 0; k < kMaxDims; ++k) {
    d.out_shape[k] = d.red_shape[k] = 1;
    d.in_strides_kept[k] = d.in_strides_red[k] = 0;
  }
  for (int k = 0; k < ndim; ++k) {
    DTMI_CHECK(shape[k] >= 0, "dtmi_reduce_sum: negative dimension");
    int64_t st = strides ? strides[k] : cstr[k];
    if (reduce_mask[k]) {
      d.red_shape[k] = shape[k];
      d.in_strides_red[k] = st;
      nred *= shape[k];
    } else {
      d.out_shape[k] = shape[k];
      d.in_strides_kept[k] = st;
      nout *= shape[k];
    }
  }
  if (nout == 0) return DTMI_OK;
  DTMI_CHECK(out && (x || nred == 0), "dtmi_reduce_sum: NULL pointer");
  TimedLaunch tl(DTMI_FAM_OTHER, (double)(nout * nred + nout) * (dtype == DTMI_F32 ? 4 : 8));
  // contiguous input reduced over a leading run of axes: [nred, nout]
  bool lead = nred > 0;
  for (int k = 0; k < ndim && lead; ++k) {
    if (strides && shape[k] > 1 && strides[k] != cstr[k]) lead = false;
    if (k > 0 && reduce_mask[k] && !reduce_mask[k - 1]) lead = false;
  }
  const int64_t vn = dtype == DTMI_F32 ? 4 : 2;
  if (lead && nout % vn == 0 && aligned(x, 16) && aligned(out, 16)) {
    const int64_t nvec = nout / vn;
    const int grid = (int)(cdiv(nvec, 256) < 8192 ? cdiv(nvec, 256) : 8192);
    if (dtype == DTMI_F32)
      reduce_lead_kernel<float><<<grid, 256, 0, stream()>>>((float*)out, (const float*)x, nout, nred);
    else
      reduce_lead_kernel<double><<<grid, 256, 0, stream()>>>((double*)out, (const double*)x, nout, nred);
    LAUNCH_CHECK("reduce_lead_kernel");
    return DTMI_OK;
  }
  if (dtype == DTMI_F32)
    reduce_axes_kernel<float><<<grid_1d(nout, 1), 256, 0, stream()>>>((float*)out, (const float*)x, d, nout, nred);
  else
    reduce_axes_kernel<double><<<grid_1d(nout, 1), 256, 0, stream()>>>((double*)out, (const double*)x, d, nout,
                                                                        nred);
  LAUNCH_CHECK("reduce_axes_kernel");
  return DTMI_OK;
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_colsum(int dtype, void* out, const void* x, int64_t rows, int64_t cols, int accumulate) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_DTYPE_OK(dtype);
  DTMI_CHECK(rows >= 0 && cols >= 0, "dtmi_colsum: negative size");
  if (cols == 0) return DTMI_OK;
  DTMI_CHECK(out != nullptr, "dtmi_colsum: NULL output");
  const size_t es = dtype == DTMI_F32 ? 4 : 8;
  if (rows == 0) {
    if (accumulate) return DTMI_OK;
    return dtmi_fill(dtype, out, 0.0, cols);
  }
  DTMI_CHECK(x != nullptr, "dtmi_colsum: NULL input");
  int64_t nparts = cdiv(rows, kColRows);
  DTMI_CHECK(nparts < 65536, "dtmi_colsum: too many rows (%lld)", (long long)rows);
  void* part = nullptr;
  int rc = pool_alloc(&part, (size_t)(nparts * cols) * es);
  if (rc) return rc;
  {
    TimedLaunch tl(DTMI_FAM_OTHER, (double)(rows * cols + cols) * es);
    dim3 g1((unsigned)cdiv(cols, 256), (unsigned)nparts);
    if (dtype == DTMI_F32) {
      colsum_stage1_kernel<float><<<g1, 256, 0, stream()>>>((float*)part, (const float*)x, rows, cols);
      launch_colreduce<float>((float*)out, (const float*)part, (int)nparts, cols, accumulate);
    } else {
      colsum_stage1_kernel<double><<<g1, 256, 0, stream()>>>((double*)part, (const double*)x, rows, cols);
      launch_colreduce<double>((double*)out, (const double*)part, (int)nparts, cols, accumulate);
    }
  }
  hipError_t le = hipGetLastError();
  pool_free(part);
  if (le != hipSuccess) return fail_hip(le, "colsum kernels", __FILE__, __LINE__);
  return DTMI_OK;
  DTMI_BODY_END
}
