// Optimizer and gradient-bucket kernels: fused AdamW (flat and multi-tensor),
// bucket flatten, rank-ordered replica average with fused sum of squares,
// deterministic sum of squares and the clip factor.
//
// All of these are HBM-bound streaming kernels: 16-byte vector loads and stores
// (4 floats / 2 doubles) when every operand is 16-byte aligned, over a grid
// that depends only on the problem size (so per-block partial sums, and
// therefore results, are the same on every run and every device). AdamW runs
// one pass of 1024-element blocks, the replica average one pass of blocks of
// four vectors per thread, both with non-temporal accesses; the multi-tensor
// kernels walk 32768-element chunks.
//
// Bit-exactness: this file is compiled with -ffp-contract=off and every update
// below is written as the same sequence of IEEE operations NumPy performs for
// dtrain's expressions, so F64 (and F32) results equal NumPy's bit for bit.
#include <cmath>
#include <vector>

#include <type_traits>

#include "common.h"

namespace dtmi {

template <typename T>
struct V16;
template <>
struct V16<float> {
  typedef float type __attribute__((ext_vector_type(4)));
  static constexpr int N = 4;
};
template <>
struct V16<double> {
  typedef double type __attribute__((ext_vector_type(2)));
  static constexpr int N = 2;
};

template <typename T>
__device__ __forceinline__ T vget(const typename V16<T>::type& v, int i) {
  return v[i];
}
template <typename T>
__device__ __forceinline__ void vset(typename V16<T>::type& v, int i, T x) {
  v[i] = x;
}

// Streaming accesses of data touched once per kernel: non-temporal loads and
// stores (measured fastest for these one-pass kernels on MI355X HBM).
template <typename V>
__device__ __forceinline__ V ld_nt(const V* p) {
  return __builtin_nontemporal_load(p);
}
template <typename V>
__device__ __forceinline__ void st_nt(V v, V* p) {
  __builtin_nontemporal_store(v, p);
}

// One-pass kernels over n elements use blocks of kBlockElems consecutive
// elements (256 threads x 16 bytes for float32, 2 x 16 bytes for float64):
// every load of a block is issued at once and blocks retire after one pass.
// The grid is a function of n alone, so per-block partial sums are too.
constexpr int64_t kBlockElems = 1024;

static int64_t onepass_grid(int64_t n) { return n > 0 ? (n + kBlockElems - 1) / kBlockElems : 1; }

// --------------------------------------------------------------- AdamW
template <typename T>
struct AdamWScalars {
  T lr, b1, b2, eps, wd, c1, c2, b1t, b2t, gscale;
};

template <typename T>
static AdamWScalars<T> make_scalars(double lr, double b1, double b2, double eps, double wd, double c1, double c2,
                                    double b1t, double b2t, double gscale) {
  // Host rounding double -> T (round to nearest), as NumPy does for a weak
  // Python float meeting an array of dtype T.
  return AdamWScalars<T>{(T)lr, (T)b1, (T)b2, (T)eps, (T)wd, (T)c1, (T)c2, (T)b1t, (T)b2t, (T)gscale};
}

// dtrain/optim.py:28-33, one element, in NumPy's operation order:
//   g = g * s                                  (train.py:159, the clip pre-scale)
//   m *= b1 ; m += (1 - b1) * g
//   v *= b2 ; v += (1 - b2) * (g * g)
//   p -= lr * (wd * p)
//   p -= lr * (m / b1t) / (sqrt(v / b2t) + eps)
template <typename T>
__device__ __forceinline__ void adamw_elem(T& p, T g, T& m, T& v, const AdamWScalars<T>& s, T gs) {
  g = g * gs;
  m = m * s.b1;
  T t1 = s.c1 * g;
  m = m + t1;
  v = v * s.b2;
  T gg = g * g;
  T t2 = s.c2 * gg;
  v = v + t2;
  T d = s.wd * p;
  d = s.lr * d;
  p = p - d;
  T mh = m / s.b1t;
  T num = s.lr * mh;
  T vh = v / s.b2t;
  T den = sqrt(vh);
  den = den + s.eps;
  T step = num / den;
  p = p - step;
}

template <typename T>
__device__ __forceinline__ T load_gscale(const AdamWScalars<T>& s, const double* gdev) {
  return gdev ? (T)(*gdev) : s.gscale;
}

template <typename T, bool VEC>
__global__ void __launch_bounds__(256) adamw_flat_kernel(T* __restrict__ p, const T* __restrict__ g,
                                                          T* __restrict__ m, T* __restrict__ v, int64_t n,
                                                          AdamWScalars<T> s, const double* gdev) {
  const T gs = load_gscale(s, gdev);
  const int64_t base = (int64_t)blockIdx.x * kBlockElems;
  if (VEC) {
    using VT = typename V16<T>::type;
    constexpr int N = V16<T>::N;
    constexpr int PER = kBlockElems / 256 / N;  // vectors per thread
    VT P[PER], G[PER], M[PER], W[PER];
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int64_t e0 = base + (int64_t)(u * 256 + threadIdx.x) * N;
      if (e0 + N <= n) {
        const int64_t k = e0 / N;
        P[u] = ld_nt(reinterpret_cast<const VT*>(p) + k);
        G[u] = ld_nt(reinterpret_cast<const VT*>(g) + k);
        M[u] = ld_nt(reinterpret_cast<const VT*>(m) + k);
        W[u] = ld_nt(reinterpret_cast<const VT*>(v) + k);
      }
    }
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int64_t e0 = base + (int64_t)(u * 256 + threadIdx.x) * N;
      if (e0 + N <= n) {
#pragma unroll
        for (int e = 0; e < N; ++e) {
          T pe = vget<T>(P[u], e), me = vget<T>(M[u], e), ve = vget<T>(W[u], e);
          adamw_elem<T>(pe, vget<T>(G[u], e), me, ve, s, gs);
          vset<T>(P[u], e, pe);
          vset<T>(M[u], e, me);
          vset<T>(W[u], e, ve);
        }
        const int64_t k = e0 / N;
        st_nt(P[u], reinterpret_cast<VT*>(p) + k);
        st_nt(M[u], reinterpret_cast<VT*>(m) + k);
        st_nt(W[u], reinterpret_cast<VT*>(v) + k);
      } else if (e0 < n) {
        for (int64_t k = e0; k < n; ++k) adamw_elem<T>(p[k], g[k], m[k], v[k], s, gs);  // ragged end
      }
    }
  } else {
    for (int64_t k = base + threadIdx.x; k < base + kBlockElems && k < n; k += 256)
      adamw_elem<T>(p[k], g[k], m[k], v[k], s, gs);
  }
}

template <typename T>
static int launch_adamw_flat(void* p, const void* g, void* m, void* v, int64_t n, const AdamWScalars<T>& s,
                             const double* gdev) {
  bool vec = aligned(p, 16) && aligned(g, 16) && aligned(m, 16) && aligned(v, 16);
  const int64_t grid = onepass_grid(n);
  DTMI_CHECK(grid < (1LL << 31), "dtmi_adamw: too many elements");
  TimedLaunch tl(DTMI_FAM_ADAMW, 7.0 * (double)n * sizeof(T));
  if (vec)
    adamw_flat_kernel<T, true><<<(unsigned)grid, 256, 0, stream()>>>((T*)p, (const T*)g, (T*)m, (T*)v, n, s, gdev);
  else
    adamw_flat_kernel<T, false><<<(unsigned)grid, 256, 0, stream()>>>((T*)p, (const T*)g, (T*)m, (T*)v, n, s,
                                                                       gdev);
  LAUNCH_CHECK("adamw_flat_kernel");
  return DTMI_OK;
}

// Multi-tensor table: one entry per tensor; chunk c of the launch belongs to
// the entry e with e.chunk_begin <= c < next.chunk_begin.
constexpr int64_t kChunk = 32768;
// Pointers read from a table in device memory are generic (flat) pointers to
// the compiler; flat accesses also count on the LDS/scalar counter, so every
// wait for them is a full wait. Casting them to the global address space
// gives global loads and stores that can be in flight together.
template <typename X>
using global_t = __attribute__((address_space(1))) X;

struct MTAdamEntry {
  void* p;
  const void* g;
  void* m;
  void* v;
  int64_t n;
  int64_t chunk_begin;
  int64_t vec;
};

__device__ __forceinline__ int find_entry(const int64_t* begins, int stride_i64, int count, int64_t c) {
  // largest e with begins[e * stride] <= c (entries sorted by chunk_begin)
  int lo = 0, hi = count - 1;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if (begins[(int64_t)mid * stride_i64] <= c)
      lo = mid;
    else
      hi = mid - 1;
  }
  return lo;
}

template <typename T>
__global__ void __launch_bounds__(256) adamw_multi_kernel(const MTAdamEntry* __restrict__ tab, int count,
                                                           AdamWScalars<T> s, const double* gdev) {
  const int64_t c = blockIdx.x;
  const int e = find_entry(&tab[0].chunk_begin, sizeof(MTAdamEntry) / sizeof(int64_t), count, c);
  const MTAdamEntry ent = tab[e];
  const T gs = load_gscale(s, gdev);
  const int64_t lo = (c - ent.chunk_begin) * kChunk;
  const int64_t hi = lo + kChunk < ent.n ? lo + kChunk : ent.n;
  T* p = (T*)ent.p;
  const T* g = (const T*)ent.g;
  T* m = (T*)ent.m;
  T* v = (T*)ent.v;
  if (ent.vec) {
    using VT = typename V16<T>::type;
    constexpr int N = V16<T>::N;
    // lo is a multiple of kChunk (a multiple of N); only the last chunk has a tail.
    const int64_t nv = (hi - lo) / N;
    global_t<VT>* pv = (global_t<VT>*)(p + lo);
    global_t<const VT>* gv = (global_t<const VT>*)(g + lo);
    global_t<VT>* mv = (global_t<VT>*)(m + lo);
    global_t<VT>* vv = (global_t<VT>*)(v + lo);
    for (int64_t i = threadIdx.x; i < nv; i += blockDim.x) {
      VT P = pv[i], G = gv[i], M = mv[i], W = vv[i];
#pragma unroll
      for (int el = 0; el < N; ++el) {
        T pe = vget<T>(P, el), me = vget<T>(M, el), ve = vget<T>(W, el);
        adamw_elem<T>(pe, vget<T>(G, el), me, ve, s, gs);
        vset<T>(P, el, pe);
        vset<T>(M, el, me);
        vset<T>(W, el, ve);
      }
      pv[i] = P;
      mv[i] = M;
      vv[i] = W;
    }
    for (int64_t k = lo + nv * N + threadIdx.x; k < hi; k += blockDim.x) adamw_elem<T>(p[k], g[k], m[k], v[k], s, gs);
  } else {
    for (int64_t k = lo + threadIdx.x; k < hi; k += blockDim.x) adamw_elem<T>(p[k], g[k], m[k], v[k], s, gs);
  }
}

// ------------------------------------------------------------- flatten
struct FlatEntry {
  const void* src;  // NULL: write zeros
  int64_t n;
  int64_t dst_off;
  int64_t chunk_begin;
  int64_t vec;
};

template <typename T>
__global__ void __launch_bounds__(256) flatten_kernel(T* __restrict__ dst, const FlatEntry* __restrict__ tab,
                                                       int count) {
  const int64_t c = blockIdx.x;
  const int e = find_entry(&tab[0].chunk_begin, sizeof(FlatEntry) / sizeof(int64_t), count, c);
  const FlatEntry ent = tab[e];
  const int64_t lo = (c - ent.chunk_begin) * kChunk;
  const int64_t hi = lo + kChunk < ent.n ? lo + kChunk : ent.n;
  const T* src = (const T*)ent.src;
  T* out = dst + ent.dst_off;
  if (ent.vec) {
    using VT = typename V16<T>::type;
    constexpr int N = V16<T>::N;
    const int64_t nv = (hi - lo) / N;
    VT* ov = reinterpret_cast<VT*>(out + lo);
    if (src) {
      // four vectors in flight per thread
      global_t<const VT>* sv = (global_t<const VT>*)(src + lo);
      int64_t i = threadIdx.x;
      for (; i + 3 * 256 < nv; i += 4 * 256) {
        VT a[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) a[u] = sv[i + u * 256];
#pragma unroll
        for (int u = 0; u < 4; ++u) ov[i + u * 256] = a[u];
      }
      for (; i < nv; i += 256) ov[i] = sv[i];
    } else {
      VT z;
      for (int el = 0; el < N; ++el) vset<T>(z, el, T(0));
      for (int64_t i = threadIdx.x; i < nv; i += blockDim.x) ov[i] = z;
    }
    for (int64_t k = lo + nv * N + threadIdx.x; k < hi; k += blockDim.x) out[k] = src ? src[k] : T(0);
  } else {
    for (int64_t k = lo + threadIdx.x; k < hi; k += blockDim.x) out[k] = src ? src[k] : T(0);
  }
}

// ------------------------------------------------------ block reduction
// Deterministic sum of one double per thread across a 256-thread block:
// butterfly within each wave (fixed pattern), then wave results in order.
__device__ __forceinline__ double block_sum_256(double x, double* lds4) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off, 64);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) lds4[wave] = x;
  __syncthreads();
  double r = 0.0;
  if (threadIdx.x == 0) r = ((lds4[0] + lds4[1]) + lds4[2]) + lds4[3];
  return r;
}

template <typename T>
__device__ __forceinline__ double sq64(T x) {
  double d = (double)x;
  return d * d;
}

// ------------------------------------------------- fixed-order average
// out[i] = (((rep_a[i] + rep_b[i]) + ...) + rep_z[i]) * inv, where the ranks
// a, b, ..., z are first, first + 1, ..., first - 1 (mod W) and `first` is the
// rank order's start for the segment holding element i: 0 everywhere for
// dtrain's direct all-reduce (comm.py:374-391); for its ring all-reduce
// (comm.py:292-303, 342-372) chunk c of a bucket buffer is summed starting at
// rank c. Segments are contiguous ranges of out given by value (at most
// kMaxSegs per launch); a block inside one segment reads its replica rows in
// that segment's rank order, so the vector path is the same for every order.
// With SUMSQ the block's float64 sum of out^2 goes to partials[blockIdx.x]
// (fixed pattern). WC > 0 fixes the replica count at compile time (the vector
// path then loads all replicas at once); WC = 0 takes it from `world`.
constexpr int kMaxSegs = 16;
// Vectors per thread of the average's blocks: 4 (all of a block's loads in
// flight at once) for arrays of at least 4M elements, else 1 (more blocks).
constexpr int64_t kAvgWideFrom = (int64_t)1 << 22;
template <typename T>
constexpr int64_t avg_elems(int per) {
  return 256 * per * (16 / (int64_t)sizeof(T));
}
// Segments of one launch: start[j] (start[0] = 0; entries past nseg hold
// INT32_MAX, so every test below ignores them without a count) and the first
// rank of each, packed four to a word. Read with compile-time indices only,
// so the table stays in scalar registers.
struct RankSegs {
  int32_t start[kMaxSegs];
  uint32_t first4[kMaxSegs / 4];
};
__device__ __forceinline__ int seg_rank(const RankSegs& sg, int j) { return (sg.first4[j >> 2] >> (8 * (j & 3))) & 0xFF; }

// The first rank of element k's segment.
__device__ __forceinline__ int seg_first(const RankSegs& sg, int64_t k) {
  int f = seg_rank(sg, 0);
#pragma unroll
  for (int j = 1; j < kMaxSegs; ++j)
    if (k >= sg.start[j]) f = seg_rank(sg, j);
  return f;
}

template <typename T, bool VEC, bool SUMSQ, int WC, bool ROT, int PER>
__global__ void __launch_bounds__(256) bucket_average_kernel(T* __restrict__ out, const T* __restrict__ rep,
                                                              int world, int64_t n, int64_t stride, T inv,
                                                              double* __restrict__ partials, RankSegs sg) {
  __shared__ double lds[4];
  constexpr int64_t kAvgElems = avg_elems<T>(PER);
  const int64_t base = (int64_t)blockIdx.x * kAvgElems;
  // rank order of the block: uniform when the block lies in one segment
  int bfirst = 0;
  bool mixed = false;
  if (ROT) {
    const int64_t bend = base + kAvgElems < n ? base + kAvgElems : n;
    bfirst = seg_rank(sg, 0);
#pragma unroll
    for (int j = 1; j < kMaxSegs; ++j) {
      const int64_t st = sg.start[j];
      if (st <= base) bfirst = seg_rank(sg, j);
      mixed = mixed || (st > base && st < bend);  // a segment boundary strictly inside the block
    }
  }
  // replica row of position r in the block's order
  auto row = [&](int r) {
    int q = bfirst + r;
    q = q >= world ? q - world : q;
    return rep + (int64_t)q * stride;
  };
  // element k in its own segment's order (blocks that straddle segments)
  auto elem = [&](int64_t k) {
    const int f = ROT && mixed ? seg_first(sg, k) : bfirst;
    T a = rep[(int64_t)f * stride + k];
    for (int r = 1; r < world; ++r) {
      int q = f + r;
      q = q >= world ? q - world : q;
      a = a + rep[(int64_t)q * stride + k];
    }
    return a;
  };
  double acc = 0.0;
  if (VEC && (WC > 0 || !(ROT && mixed))) {
    using VT = typename V16<T>::type;
    constexpr int N = V16<T>::N;
    if constexpr (WC > 0) {
      // WC replicas known at compile time: every load of the block is issued
      // before the first add (rows in rank order 0..W-1, so no load waits for
      // the segment lookup), and the adds follow the block's rank order
      VT v[PER][WC];
#pragma unroll
      for (int u = 0; u < PER; ++u) {
        const int64_t e0 = base + (int64_t)(u * 256 + threadIdx.x) * N;
        if (e0 + N <= n)
#pragma unroll
          for (int r = 0; r < WC; ++r) v[u][r] = ld_nt(reinterpret_cast<const VT*>(rep + (int64_t)r * stride) + e0 / N);
      }
      // ((v_f + v_{f+1}) + ...) + v_{f-1}: one compile-time order per first rank
      auto ordered_sum = [&](const VT(&x)[WC]) {
        VT a = x[0];
        auto fold = [&](auto fc) {
          constexpr int F = decltype(fc)::value;
          a = x[F];
#pragma unroll
          for (int r = 1; r < WC; ++r) a = a + x[(F + r) % WC];
        };
        if (!ROT) {
          fold(std::integral_constant<int, 0>{});
        } else {
          switch (bfirst) {
            case 0: fold(std::integral_constant<int, 0>{}); break;
            case 1: fold(std::integral_constant<int, 1 % WC>{}); break;
            case 2: fold(std::integral_constant<int, 2 % WC>{}); break;
            default: fold(std::integral_constant<int, 3 % WC>{}); break;
          }
        }
        return a;
      };
      // a block across a segment edge: each element in its own segment's
      // order (every order is summed, the element's is kept)
      auto mixed_sum = [&](const VT(&x)[WC], int64_t e0) {
        VT a;
#pragma unroll
        for (int e = 0; e < N; ++e) {
          const int f = seg_first(sg, e0 + e);
          T pick = T(0);
#pragma unroll
          for (int F = 0; F < WC; ++F) {
            T t = vget<T>(x[F], e);
#pragma unroll
            for (int r = 1; r < WC; ++r) t = t + vget<T>(x[(F + r) % WC], e);
            pick = f == F ? t : pick;
          }
          vset<T>(a, e, pick);
        }
        return a;
      };
#pragma unroll
      for (int u = 0; u < PER; ++u) {
        const int64_t e0 = base + (int64_t)(u * 256 + threadIdx.x) * N;
        if (e0 + N <= n) {
          VT a = ROT && mixed ? mixed_sum(v[u], e0) : ordered_sum(v[u]);
          a = a * inv;
          if (SUMSQ)
#pragma unroll
            for (int e = 0; e < N; ++e) acc += sq64(vget<T>(a, e));
          st_nt(a, reinterpret_cast<VT*>(out) + e0 / N);
        } else if (e0 < n) {
          for (int64_t k = e0; k < n; ++k) {  // ragged end
            T o = elem(k) * inv;
            out[k] = o;
            if (SUMSQ) acc += sq64(o);
          }
        }
      }
    } else {
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int64_t e0 = base + (int64_t)(u * 256 + threadIdx.x) * N;
      if (e0 + N <= n) {
        const int64_t k = e0 / N;
        VT a;
        {
          a = ld_nt(reinterpret_cast<const VT*>(row(0)) + k);
          for (int r = 1; r < world; ++r) a = a + ld_nt(reinterpret_cast<const VT*>(row(r)) + k);
        }
        a = a * inv;
        if (SUMSQ)
#pragma unroll
          for (int e = 0; e < N; ++e) acc += sq64(vget<T>(a, e));
        st_nt(a, reinterpret_cast<VT*>(out) + k);
      } else if (e0 < n) {
        for (int64_t k = e0; k < n; ++k) {  // ragged end
          T o = elem(k) * inv;
          out[k] = o;
          if (SUMSQ) acc += sq64(o);
        }
      }
    }
    }
  } else {
    for (int64_t k = base + threadIdx.x; k < base + kAvgElems && k < n; k += 256) {
      T o = elem(k) * inv;
      out[k] = o;
      if (SUMSQ) acc += sq64(o);
    }
  }
  if (SUMSQ) {
    double b = block_sum_256(acc, lds);
    if (threadIdx.x == 0) partials[blockIdx.x] = b;
  }
}

template <typename T>
static int average_grid(int64_t n) {
  const int64_t e = avg_elems<T>(n >= kAvgWideFrom ? 4 : 1);
  return n > 0 ? (int)((n + e - 1) / e) : 1;
}

// -------------------------------------------------------- sum of squares
struct SumsqEntry {
  const void* p;
  int64_t n;
  int64_t chunk_begin;
  int64_t vec;
};

template <typename T>
__global__ void __launch_bounds__(256) sumsq_multi_kernel(const SumsqEntry* __restrict__ tab, int count,
                                                           double* __restrict__ partials) {
  __shared__ double lds[4];
  const int64_t c = blockIdx.x;
  const int e = find_entry(&tab[0].chunk_begin, sizeof(SumsqEntry) / sizeof(int64_t), count, c);
  const SumsqEntry ent = tab[e];
  const int64_t lo = (c - ent.chunk_begin) * kChunk;
  const int64_t hi = lo + kChunk < ent.n ? lo + kChunk : ent.n;
  const T* x = (const T*)ent.p;
  double acc = 0.0;
  if (ent.vec) {
    using VT = typename V16<T>::type;
    constexpr int N = V16<T>::N;
    const int64_t nv = (hi - lo) / N;
    global_t<const VT>* xv = (global_t<const VT>*)(x + lo);
    // four vectors are loaded ahead; the squares are added in the same
    // element order as a one-vector loop
    int64_t i = threadIdx.x;
    for (; i + 3 * 256 < nv; i += 4 * 256) {
      VT a[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) a[u] = xv[i + u * 256];
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int el = 0; el < N; ++el) acc += sq64(vget<T>(a[u], el));
    }
    for (; i < nv; i += 256) {
      VT a = xv[i];
#pragma unroll
      for (int el = 0; el < N; ++el) acc += sq64(vget<T>(a, el));
    }
    for (int64_t k = lo + nv * N + threadIdx.x; k < hi; k += 256) acc += sq64(x[k]);
  } else {
    for (int64_t k = lo + threadIdx.x; k < hi; k += blockDim.x) acc += sq64(x[k]);
  }
  double b = block_sum_256(acc, lds);
  if (threadIdx.x == 0) partials[c] = b;
}

// One block of 1024 threads sums `count` partials: thread t adds partials
// t, t+1024, ... in order, then a fixed tree.
__global__ void __launch_bounds__(1024) sumsq_finish_kernel(const double* __restrict__ partials, int64_t count,
                                                             double* __restrict__ out, int accumulate) {
  __shared__ double lds[16];
  double acc = 0.0;
  for (int64_t i = threadIdx.x; i < count; i += 1024) acc += partials[i];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    double r = 0.0;
    for (int w = 0; w < 16; ++w) r += lds[w];
    *out = accumulate ? *out + r : r;
  }
}

__global__ void clip_scale_kernel(const double* sq, double max_norm, double* scale, double* norm) {
  double n = sqrt(*sq);
  double s = (n <= max_norm || n == 0.0) ? 1.0 : max_norm / (n + 1e-6);
  *scale = s;
  if (norm) *norm = n;
}

}  // namespace dtmi

using namespace dtmi;

DTMI_EXPORT int dtmi_adamw(int dtype, void* p, const void* g, void* m, void* v, int64_t n, double lr, double b1,
                           double b2, double eps, double wd, double c1, double c2, double b1t, double b2t,
                           double gscale, const double* gscale_dev) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_DTYPE_OK(dtype);
  DTMI_CHECK(n >= 0, "dtmi_adamw: negative size");
  if (n == 0) return DTMI_OK;
  DTMI_CHECK(p && g && m && v, "dtmi_adamw: NULL pointer");
  if (dtype == DTMI_F32)
    return launch_adamw_flat<float>(p, g, m, v, n, make_scalars<float>(lr, b1, b2, eps, wd, c1, c2, b1t, b2t, gscale),
                                    gscale_dev);
  return launch_adamw_flat<double>(p, g, m, v, n, make_scalars<double>(lr, b1, b2, eps, wd, c1, c2, b1t, b2t, gscale),
                                   gscale_dev);
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_adamw_multi(int dtype, int ntensors, void* const* p, const void* const* g, void* const* m,
                                 void* const* v, const int64_t* n, double lr, double b1, double b2, double eps,
                                 double wd, double c1, double c2, double b1t, double b2t, double gscale,
                                 const double* gscale_dev) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_DTYPE_OK(dtype);
  DTMI_CHECK(ntensors >= 0, "dtmi_adamw_multi: negative tensor count");
  DTMI_CHECK(ntensors == 0 || (p && g && m && v && n), "dtmi_adamw_multi: NULL table");
  const size_t es = dtype == DTMI_F32 ? 4 : 8;
  std::vector<MTAdamEntry> tab;
  tab.reserve(ntensors);
  int64_t chunks = 0;
  double bytes = 0;
  for (int i = 0; i < ntensors; ++i) {
    DTMI_CHECK(n[i] >= 0, "dtmi_adamw_multi: tensor %d has negative size", i);
    if (g[i] == nullptr || n[i] == 0) continue;  // optim.py:26-27: no gradient, no update
    DTMI_CHECK(p[i] && m[i] && v[i], "dtmi_adamw_multi: tensor %d has a NULL p/m/v", i);
    bool vec = aligned(p[i], 16) && aligned(g[i], 16) && aligned(m[i], 16) && aligned(v[i], 16);
    tab.push_back(MTAdamEntry{p[i], g[i], m[i], v[i], n[i], chunks, vec ? 1 : 0});
    chunks += cdiv(n[i], kChunk);
    bytes += 7.0 * (double)n[i] * es;
  }
  if (tab.empty()) return DTMI_OK;
  DTMI_CHECK(chunks < (int64_t)1 << 31, "dtmi_adamw_multi: too many chunks");
  void* dtab = nullptr;
  int rc = upload_table(tab.data(), tab.size() * sizeof(MTAdamEntry), &dtab);
  if (rc) return rc;
  {
    TimedLaunch tl(DTMI_FAM_ADAMW, bytes);
    if (dtype == DTMI_F32)
      adamw_multi_kernel<float><<<(unsigned)chunks, 256, 0, stream()>>>(
          (const MTAdamEntry*)dtab, (int)tab.size(), make_scalars<float>(lr, b1, b2, eps, wd, c1, c2, b1t, b2t, gscale),
          gscale_dev);
    else
      adamw_multi_kernel<double><<<(unsigned)chunks, 256, 0, stream()>>>(
          (const MTAdamEntry*)dtab, (int)tab.size(),
          make_scalars<double>(lr, b1, b2, eps, wd, c1, c2, b1t, b2t, gscale), gscale_dev);
  }
  hipError_t le = hipGetLastError();
  pool_free(dtab);
  if (le != hipSuccess) return fail_hip(le, "adamw_multi_kernel", __FILE__, __LINE__);
  return DTMI_OK;
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_bucket_flatten(int dtype, void* dst, const void* const* srcs, const int64_t* counts, int nsrc) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_DTYPE_OK(dtype);
  DTMI_CHECK(nsrc >= 0, "dtmi_bucket_flatten: negative source count");
  if (nsrc == 0) return DTMI_OK;
  DTMI_CHECK(dst && srcs && counts, "dtmi_bucket_flatten: NULL argument");
  const size_t es = dtype == DTMI_F32 ? 4 : 8;
  std::vector<FlatEntry> tab;
  tab.reserve(nsrc);
  int64_t off = 0, chunks = 0;
  double bytes = 0;
  for (int i = 0; i < nsrc; ++i) {
    DTMI_CHECK(counts[i] >= 0, "dtmi_bucket_flatten: source %d has negative size", i);
    if (counts[i] > 0) {
      char* d = static_cast<char*>(dst) + off * es;
      bool vec = aligned(d, 16) && (srcs[i] == nullptr || aligned(srcs[i], 16));
      tab.push_back(FlatEntry{srcs[i], counts[i], off, chunks, vec ? 1 : 0});
      chunks += cdiv(counts[i], kChunk);
      bytes += (srcs[i] ? 2.0 : 1.0) * (double)counts[i] * es;
    }
    off += counts[i];
  }
  if (tab.empty()) return DTMI_OK;
  DTMI_CHECK(chunks < (int64_t)1 << 31, "dtmi_bucket_flatten: too many chunks");
  void* dtab = nullptr;
  int rc = upload_table(tab.data(), tab.size() * sizeof(FlatEntry), &dtab);
  if (rc) return rc;
  {
    TimedLaunch tl(DTMI_FAM_FLATTEN, bytes);
    if (dtype == DTMI_F32)
      flatten_kernel<float><<<(unsigned)chunks, 256, 0, stream()>>>((float*)dst, (const FlatEntry*)dtab,
                                                                    (int)tab.size());
    else
      flatten_kernel<double><<<(unsigned)chunks, 256, 0, stream()>>>((double*)dst, (const FlatEntry*)dtab,
                                                                     (int)tab.size());
  }
  hipError_t le = hipGetLastError();
  pool_free(dtab);
  if (le != hipSuccess) return fail_hip(le, "flatten_kernel", __FILE__, __LINE__);
  return DTMI_OK;
  DTMI_BODY_END
}

template <typename T, bool ROT, int PER>
static void launch_average_p(int grid, T* O, const T* R, int world, int64_t n, int64_t stride, T inv,
                             double* partials, const RankSegs& sg, bool vec) {
  if (vec) {
    auto go = [&](auto wc) {
      constexpr int WC = decltype(wc)::value;
      if (partials)
        bucket_average_kernel<T, true, true, WC, ROT, PER>
            <<<grid, 256, 0, stream()>>>(O, R, world, n, stride, inv, partials, sg);
      else
        bucket_average_kernel<T, true, false, WC, ROT, PER>
            <<<grid, 256, 0, stream()>>>(O, R, world, n, stride, inv, partials, sg);
    };
    switch (world) {
      case 2: go(std::integral_constant<int, 2>{}); break;
      case 3: go(std::integral_constant<int, 3>{}); break;
      case 4: go(std::integral_constant<int, 4>{}); break;
      default: go(std::integral_constant<int, 0>{}); break;
    }
  } else {
    if (partials)
      bucket_average_kernel<T, false, true, 0, ROT, PER><<<grid, 256, 0, stream()>>>(O, R, world, n, stride, inv,
                                                                                      partials, sg);
    else
      bucket_average_kernel<T, false, false, 0, ROT, PER><<<grid, 256, 0, stream()>>>(O, R, world, n, stride, inv,
                                                                                       partials, sg);
  }
}

template <typename T, bool ROT>
static int launch_average_t(void* out, const void* rep, int world, int64_t n, int64_t stride, double inv_w,
                            double* partials, const RankSegs& sg) {
  bool vec = aligned(out, 16) && aligned(rep, 16) && ((stride * (int64_t)sizeof(T)) % 16 == 0);
  int grid = average_grid<T>(n);
  T inv = (T)inv_w;
  T* O = (T*)out;
  const T* R = (const T*)rep;
  if (n >= kAvgWideFrom)
    launch_average_p<T, ROT, 4>(grid, O, R, world, n, stride, inv, partials, sg, vec);
  else
    launch_average_p<T, ROT, 1>(grid, O, R, world, n, stride, inv, partials, sg, vec);
  LAUNCH_CHECK("bucket_average_kernel");
  return DTMI_OK;
}

// One launch per run of at most kMaxSegs segments, each over its own element
// range (sum-of-squares partials are taken only with a single launch).
template <typename T>
static int launch_average(void* out, const void* rep, int world, int64_t n, int64_t stride, double inv_w,
                          double* partials, const int64_t* seg_start, const int* seg_first, int nseg) {
  TimedLaunch tl(DTMI_FAM_BUCKET_AVG, (double)(world + 1) * (double)n * sizeof(T));
  RankSegs sg{};
  for (int j = 0; j < kMaxSegs; ++j) sg.start[j] = INT32_MAX;
  bool rot = false;
  for (int s = 0; s < nseg; ++s) rot = rot || seg_first[s] != 0;
  if (!rot || world <= 2) {  // one order for all (for W <= 2 every order gives the same bits)
    sg.start[0] = 0;
    return launch_average_t<T, false>(out, rep, world, n, stride, inv_w, partials, sg);
  }
  int s0 = 0;
  while (s0 < nseg) {
    const int cnt = nseg - s0 < kMaxSegs ? nseg - s0 : kMaxSegs;
    const int64_t lo = seg_start[s0], hi = s0 + cnt < nseg ? seg_start[s0 + cnt] : n;
    DTMI_CHECK(hi - lo < INT32_MAX, "dtmi_bucket_average_ring: a run of %d segments spans %lld elements (< 2^31)",
               cnt, (long long)(hi - lo));
    for (int j = 0; j < kMaxSegs; ++j) sg.start[j] = INT32_MAX;
    for (int j = 0; j < kMaxSegs / 4; ++j) sg.first4[j] = 0;
    for (int j = 0; j < cnt; ++j) {
      sg.start[j] = (int32_t)(seg_start[s0 + j] - lo);
      sg.first4[j >> 2] |= (uint32_t)seg_first[s0 + j] << (8 * (j & 3));
    }
    int rc = launch_average_t<T, true>((T*)out + lo, (const T*)rep + lo, world, hi - lo, stride, inv_w, partials, sg);
    if (rc) return rc;
    s0 += cnt;
  }
  return DTMI_OK;
}

static int check_average(int world, int64_t n, const void* out, const void* replicas, int64_t replica_stride,
                         const char* who) {
  DTMI_CHECK(world >= 1, "%s: world must be >= 1 (got %d)", who, world);
  DTMI_CHECK(out && replicas, "%s: NULL pointer", who);
  DTMI_CHECK(world == 1 || replica_stride >= n, "%s: replica_stride %lld < n %lld", who, (long long)replica_stride,
             (long long)n);
  return DTMI_OK;
}

DTMI_EXPORT int dtmi_bucket_average(int dtype, void* out, const void* replicas, int world, int64_t n,
                                    int64_t replica_stride, double inv_w, double* sumsq_partials, int64_t* nblocks) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_DTYPE_OK(dtype);
  DTMI_CHECK(n >= 0, "dtmi_bucket_average: negative size");
  if (nblocks) *nblocks = n > 0 ? (dtype == DTMI_F32 ? average_grid<float>(n) : average_grid<double>(n)) : 0;
  if (sumsq_partials == nullptr && nblocks != nullptr && out == nullptr) return DTMI_OK;  // size query
  if (n == 0) return DTMI_OK;
  int rc = check_average(world, n, out, replicas, replica_stride, "dtmi_bucket_average");
  if (rc) return rc;
  const int64_t s0 = 0;
  const int f0 = 0;
  if (dtype == DTMI_F32)
    return launch_average<float>(out, replicas, world, n, replica_stride, inv_w, sumsq_partials, &s0, &f0, 1);
  return launch_average<double>(out, replicas, world, n, replica_stride, inv_w, sumsq_partials, &s0, &f0, 1);
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_bucket_average_ring(int dtype, void* out, const void* replicas, int world, int64_t n,
                                         int64_t replica_stride, double inv_w, const int64_t* seg_start,
                                         const int* seg_first, int nseg, double* sumsq_partials) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_DTYPE_OK(dtype);
  DTMI_CHECK(n >= 0, "dtmi_bucket_average_ring: negative size");
  if (n == 0) return DTMI_OK;
  int rc = check_average(world, n, out, replicas, replica_stride, "dtmi_bucket_average_ring");
  if (rc) return rc;
  DTMI_CHECK(nseg >= 1 && seg_start && seg_first, "dtmi_bucket_average_ring: need at least one segment");
  DTMI_CHECK(seg_start[0] == 0, "dtmi_bucket_average_ring: the first segment must start at 0");
  for (int s = 0; s < nseg; ++s) {
    DTMI_CHECK(seg_first[s] >= 0 && seg_first[s] < world && seg_first[s] < 256,
               "dtmi_bucket_average_ring: segment %d starts at rank %d", s, seg_first[s]);
    DTMI_CHECK((s + 1 < nseg ? seg_start[s + 1] : n) > seg_start[s],
               "dtmi_bucket_average_ring: segment starts must increase inside [0, n)");
  }
  DTMI_CHECK(sumsq_partials == nullptr || nseg <= kMaxSegs,
             "dtmi_bucket_average_ring: sum-of-squares partials need at most %d segments", kMaxSegs);
  if (dtype == DTMI_F32)
    return launch_average<float>(out, replicas, world, n, replica_stride, inv_w, sumsq_partials, seg_start,
                                 seg_first, nseg);
  return launch_average<double>(out, replicas, world, n, replica_stride, inv_w, sumsq_partials, seg_start,
                                seg_first, nseg);
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_sumsq(int dtype, const void* const* ptrs, const int64_t* counts, int nt, double* out_dev) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_DTYPE_OK(dtype);
  DTMI_CHECK(out_dev != nullptr, "dtmi_sumsq: NULL output");
  DTMI_CHECK(nt >= 0 && (nt == 0 || (ptrs && counts)), "dtmi_sumsq: bad table");
  const size_t es = dtype == DTMI_F32 ? 4 : 8;
  std::vector<SumsqEntry> tab;
  int64_t chunks = 0;
  double bytes = 0;
  for (int i = 0; i < nt; ++i) {
    DTMI_CHECK(counts[i] >= 0, "dtmi_sumsq: tensor %d has negative size", i);
    if (ptrs[i] == nullptr || counts[i] == 0) continue;
    tab.push_back(SumsqEntry{ptrs[i], counts[i], chunks, aligned(ptrs[i], 16) ? 1 : 0});
    chunks += cdiv(counts[i], kChunk);
    bytes += (double)counts[i] * es;
  }
  if (tab.empty()) {
    // empty sum = 0.0
    double zero = 0.0;
    return dtmi_memcpy_h2d(out_dev, &zero, sizeof(double));
  }
  DTMI_CHECK(chunks < (int64_t)1 << 31, "dtmi_sumsq: too many chunks");
  void* dtab = nullptr;
  int rc = upload_table(tab.data(), tab.size() * sizeof(SumsqEntry), &dtab);
  if (rc) return rc;
  void* parts = nullptr;
  rc = pool_alloc(&parts, (size_t)chunks * sizeof(double));
  if (rc) {
    pool_free(dtab);
    return rc;
  }
  {
    TimedLaunch tl(DTMI_FAM_SUMSQ, bytes);
    if (dtype == DTMI_F32)
      sumsq_multi_kernel<float><<<(unsigned)chunks, 256, 0, stream()>>>((const SumsqEntry*)dtab, (int)tab.size(),
                                                                        (double*)parts);
    else
      sumsq_multi_kernel<double><<<(unsigned)chunks, 256, 0, stream()>>>((const SumsqEntry*)dtab, (int)tab.size(),
                                                                         (double*)parts);
    sumsq_finish_kernel<<<1, 1024, 0, stream()>>>((const double*)parts, chunks, out_dev, 0);
  }
  hipError_t le = hipGetLastError();
  pool_free(dtab);
  pool_free(parts);
  if (le != hipSuccess) return fail_hip(le, "sumsq kernels", __FILE__, __LINE__);
  return DTMI_OK;
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_sumsq_finish(const double* partials, int64_t count, double* out_dev, int accumulate) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_CHECK(out_dev != nullptr, "dtmi_sumsq_finish: NULL output");
  DTMI_CHECK(count >= 0 && (count == 0 || partials), "dtmi_sumsq_finish: bad partials");
  TimedLaunch tl(DTMI_FAM_SUMSQ, (double)count * 8);
  sumsq_finish_kernel<<<1, 1024, 0, stream()>>>(partials, count, out_dev, accumulate);
  LAUNCH_CHECK("sumsq_finish_kernel");
  return DTMI_OK;
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_clip_scale(const double* sumsq_dev, double max_norm, double* scale_dev, double* norm_dev) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_CHECK(sumsq_dev && scale_dev, "dtmi_clip_scale: NULL pointer");
  clip_scale_kernel<<<1, 1, 0, stream()>>>(sumsq_dev, max_norm, scale_dev, norm_dev);
  LAUNCH_CHECK("clip_scale_kernel");
  return DTMI_OK;
  DTMI_BODY_END
}
