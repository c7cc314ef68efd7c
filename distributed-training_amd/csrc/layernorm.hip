// LayerNorm forward and backward (dtrain/autograd.py:207-223).
//
// One 64-lane wave owns one row; the row lives in registers (each lane holds
// NV 16-byte vectors, or NV scalars when the row is not vector-aligned), so x
// and dy are read from HBM exactly once and the row reductions are wave
// butterflies (no LDS, no barriers). Four waves per 256-thread block. Rows
// longer than 16 vectors per lane take a block per row instead (below).
//
// Backward fuses dx with the column reductions dgamma = sum_rows(dy * xh) and
// dbeta = sum_rows(dy): every wave accumulates its rows' contributions in
// registers, the four waves of a block combine through LDS in wave order, and
// each block writes one partial row; a second kernel sums the partial rows in
// block order. The grid depends only on the row count, so results are
// bit-reproducible.
#include <cmath>

#include "colreduce.h"
#include "common.h"
#include "rowln.h"

namespace dtmi {

template <typename T, int NV, int VW>
__global__ void __launch_bounds__(256) ln_fwd_kernel(T* __restrict__ y, T* __restrict__ mean_out,
                                                      T* __restrict__ rstd_out, const T* __restrict__ x,
                                                      const T* __restrict__ w, const T* __restrict__ b, int64_t rows,
                                                      int cols, T eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * cols;
  T xv[NV][VW];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = VW * lane + 64 * VW * j;
    if (c < cols) {
      load_vec<T, VW>(xv[j], xr + c);
    } else {
#pragma unroll
      for (int e = 0; e < VW; ++e) xv[j][e] = T(0);
    }
  }
  ln_row_fwd<T, NV, VW>(xv, cols, lane, w, b, eps, y + row * cols, mean_out + row, rstd_out + row);
}

// out = ((p_0 + p_1) + ...) + p_{n-1}, elementwise, parts `stride` apart.
template <typename T>
__global__ void __launch_bounds__(256) sum_parts_kernel(T* __restrict__ out, const T* __restrict__ parts,
                                                         int64_t stride, int n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < stride; i += (int64_t)gridDim.x * 256) {
    T v = parts[i];
    for (int p = 1; p < n; ++p) v = v + parts[(int64_t)p * stride + i];
    out[i] = v;
  }
}

// Blocks needed for the deterministic column partials: a function of rows only.
static int ln_bwd_blocks(int64_t rows) {
  int64_t b = cdiv(rows, 4 * 2);  // two rows per wave
  if (b < 1) b = 1;
  return (int)(b < 512 ? b : 512);
}

// NP > 1: dy is the in-order sum of NP split-K partials of the product that
// made it, part p at dy + p * pstride (((p0 + p1) + ...), the sum pass's
// order), summed here as the rows are loaded instead of in a pass of its own.
template <typename T, int NV, int VW, int NP = 1>
__global__ void __launch_bounds__(256) ln_bwd_kernel(T* __restrict__ dx, T* __restrict__ part_dw,
                                                      T* __restrict__ part_db, const T* __restrict__ dy,
                                                      const T* __restrict__ x, const T* __restrict__ w,
                                                      const T* __restrict__ mean, const T* __restrict__ rstd,
                                                      const T* __restrict__ addend, int64_t rows, int cols,
                                                      int accumulate_dx, int64_t pstride = 0) {
  extern __shared__ unsigned char lds_raw[];
  T* lds = reinterpret_cast<T*>(lds_raw);  // [4 waves][2][NV*VW*64]
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t wstride = (int64_t)gridDim.x * 4;
  T wv[NV][VW], adw[NV][VW], adb[NV][VW];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = VW * lane + 64 * VW * j;
#pragma unroll
    for (int e = 0; e < VW; ++e) adw[j][e] = adb[j][e] = T(0);
    if (c < cols) {
      load_vec<T, VW>(wv[j], w + c);
    } else {
#pragma unroll
      for (int e = 0; e < VW; ++e) wv[j][e] = T(0);
    }
  }
  const T n = (T)cols;
  // Software pipeline: the next row's dy, x, mean and rstd are loaded while
  // the current row is reduced and stored, so every wave keeps a row of loads
  // in flight. Rows longer than 8 vectors per lane load each vector where it
  // is used instead (a second row set would spill). The arithmetic per row is
  // the same.
  constexpr bool PF = NV <= 8;
  static_assert(NP == 1 || PF, "split-K partials: rows of up to 8 vectors per lane");
  // what dx adds to: the existing dx, or the addend (a row's own rows only,
  // so the next row's are read ahead of this row's store)
  const T* base = accumulate_dx ? dx : addend;
  T gn[NP][NV][VW], xn[NV][VW], an[NV][VW];
  T mun = T(0), rsn = T(0);
  int64_t row = (int64_t)blockIdx.x * 4 + wave;
  auto load_row = [&](int64_t r) {
    mun = mean[r];
    rsn = rstd[r];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int c = VW * lane + 64 * VW * j;
      if (c < cols) {
#pragma unroll
        for (int p = 0; p < NP; ++p) load_vec<T, VW>(gn[p][j], dy + p * pstride + r * cols + c);
        load_vec<T, VW>(xn[j], x + r * cols + c);
        if (base) load_vec<T, VW>(an[j], base + r * cols + c);
      }
    }
  };
  if (PF && row < rows) load_row(row);
  for (; row < rows; row += wstride) {
    T mu, rs;
    T gv[NV][VW], xh[NV][VW], av[NV][VW];
    if constexpr (PF) {
      mu = mun;
      rs = rsn;
#pragma unroll
      for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int e = 0; e < VW; ++e) {
          T v = gn[0][j][e];
#pragma unroll
          for (int p = 1; p < NP; ++p) v = v + gn[p][j][e];
          gv[j][e] = v;
          xh[j][e] = xn[j][e];
          av[j][e] = an[j][e];
        }
      if (row + wstride < rows) load_row(row + wstride);
    } else {
      mu = mean[row];
      rs = rstd[row];
    }
    T s1 = T(0), s2 = T(0);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int c = VW * lane + 64 * VW * j;
      if (c < cols) {
        if constexpr (!PF) {
          load_vec<T, VW>(gv[j], dy + row * cols + c);
          load_vec<T, VW>(xh[j], x + row * cols + c);
        }
#pragma unroll
        for (int e = 0; e < VW; ++e) {
          xh[j][e] = (xh[j][e] - mu) * rs;
          T gxh = gv[j][e] * wv[j][e];
          s1 += gxh;
          s2 += gxh * xh[j][e];
          adw[j][e] += gv[j][e] * xh[j][e];
          adb[j][e] += gv[j][e];
        }
      }
    }
    const T m1 = wave_sum(s1) / n;
    const T m2 = wave_sum(s2) / n;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int c = VW * lane + 64 * VW * j;
      if (c < cols) {
        // dx (+)= r: onto the existing dx, or a separate addend written to dx
        // (pending + r: the order of the backward engine's sum)
        T o[VW];
        const bool add = base != nullptr;
        if constexpr (PF) {
#pragma unroll
          for (int e = 0; e < VW; ++e) o[e] = av[j][e];
        } else {
          if (add) load_vec<T, VW>(o, base + row * cols + c);
        }
#pragma unroll
        for (int e = 0; e < VW; ++e) {
          T gxh = gv[j][e] * wv[j][e];
          T r = rs * ((gxh - m1) - xh[j][e] * m2);
          o[e] = add ? o[e] + r : r;
        }
        store_vec<T, VW>(dx + row * cols + c, o);
      }
    }
  }
  // combine the four waves in wave order, write this block's partial rows
  constexpr int PER = NV * VW;
  T* mine = lds + (size_t)wave * 2 * PER * 64;
#pragma unroll
  for (int j = 0; j < NV; ++j)
#pragma unroll
    for (int e = 0; e < VW; ++e) {
      mine[(j * VW + e) * 64 + lane] = adw[j][e];
      mine[PER * 64 + (j * VW + e) * 64 + lane] = adb[j][e];
    }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
      for (int e = 0; e < VW; ++e) {
        const int k = (j * VW + e) * 64 + lane;
        T sdw = lds[k], sdb = lds[PER * 64 + k];
#pragma unroll
        for (int wv2 = 1; wv2 < 4; ++wv2) {
          sdw += lds[(size_t)wv2 * 2 * PER * 64 + k];
          sdb += lds[(size_t)wv2 * 2 * PER * 64 + PER * 64 + k];
        }
        const int c = VW * lane + 64 * VW * j + e;
        if (c < cols) {
          part_dw[(int64_t)blockIdx.x * cols + c] = sdw;
          part_db[(int64_t)blockIdx.x * cols + c] = sdb;
        }
      }
  }
}

// ------------------------------------------------------------- wide rows
// Rows longer than a wave's registers hold (more than 16 vectors per lane):
// one 256-thread block per row, the row re-read from memory per pass (mean,
// variance, output; backward: the two row sums, then dx). Column partials of
// dgamma / dbeta: each block accumulates its rows' contributions into its own
// partial row in memory (each thread owns the same columns of every row, so
// the updates are ordered), summed in block order by the column reduction.
template <typename T>
__device__ __forceinline__ T block_sum_bcast(T x, T* red) {
  x = wave_sum(x);
  const int wave = threadIdx.x >> 6;
  __syncthreads();  // red is free (its previous values were read)
  if ((threadIdx.x & 63) == 0) red[wave] = x;
  __syncthreads();
  return ((red[0] + red[1]) + red[2]) + red[3];
}

template <typename T>
__global__ void __launch_bounds__(256) ln_fwd_wide_kernel(T* __restrict__ y, T* __restrict__ mean_out,
                                                           T* __restrict__ rstd_out, const T* __restrict__ x,
                                                           const T* __restrict__ w, const T* __restrict__ b,
                                                           int64_t rows, int64_t cols, T eps) {
  __shared__ T red[4];
  const T n = (T)cols;
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const T* xr = x + row * cols;
    T s = T(0);
    for (int64_t c = threadIdx.x; c < cols; c += 256) s += xr[c];
    const T mu = block_sum_bcast(s, red) / n;
    T q = T(0);
    for (int64_t c = threadIdx.x; c < cols; c += 256) {
      T xc = xr[c] - mu;
      q += xc * xc;
    }
    const T var = block_sum_bcast(q, red) / n;
    const T rstd = T(1) / sqrt(var + eps);
    T* yr = y + row * cols;
    for (int64_t c = threadIdx.x; c < cols; c += 256) {
      T xh = (xr[c] - mu) * rstd;
      yr[c] = xh * w[c] + b[c];
    }
    if (threadIdx.x == 0) {
      mean_out[row] = mu;
      rstd_out[row] = rstd;
    }
  }
}

template <typename T>
__global__ void __launch_bounds__(256) ln_bwd_wide_kernel(T* __restrict__ dx, T* __restrict__ part_dw,
                                                           T* __restrict__ part_db, const T* __restrict__ dy,
                                                           const T* __restrict__ x, const T* __restrict__ w,
                                                           const T* __restrict__ mean, const T* __restrict__ rstd,
                                                           const T* __restrict__ addend, int64_t rows, int64_t cols,
                                                           int accumulate_dx) {
  __shared__ T red[4];
  const T n = (T)cols;
  T* pw = part_dw + (int64_t)blockIdx.x * cols;
  T* pb = part_db + (int64_t)blockIdx.x * cols;
  for (int64_t c = threadIdx.x; c < cols; c += 256) pw[c] = pb[c] = T(0);
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const T mu = mean[row], rs = rstd[row];
    const T* xr = x + row * cols;
    const T* gr = dy + row * cols;
    T s1 = T(0), s2 = T(0);
    for (int64_t c = threadIdx.x; c < cols; c += 256) {
      const T xh = (xr[c] - mu) * rs;
      const T gxh = gr[c] * w[c];
      s1 += gxh;
      s2 += gxh * xh;
    }
    const T m1 = block_sum_bcast(s1, red) / n;
    const T m2 = block_sum_bcast(s2, red) / n;
    T* dr = dx + row * cols;
    const T* ar = addend ? addend + row * cols : nullptr;
    for (int64_t c = threadIdx.x; c < cols; c += 256) {
      const T gv = gr[c];
      const T xh = (xr[c] - mu) * rs;
      const T gxh = gv * w[c];
      const T r = rs * ((gxh - m1) - xh * m2);
      dr[c] = accumulate_dx ? dr[c] + r : (ar ? ar[c] + r : r);
      pw[c] += gv * xh;
      pb[c] += gv;
    }
  }
}

// Blocks of the wide backward: one partial row each, at most 512 and at most
// 64 MiB of partials.
static int ln_bwd_wide_blocks(int64_t rows, int64_t cols, size_t es) {
  int64_t b = rows < 512 ? rows : 512;
  const int64_t cap = ((int64_t)64 << 20) / (2 * cols * (int64_t)es);
  if (b > cap) b = cap;
  return (int)(b < 1 ? 1 : b);
}

// ---------------------------------------------------------------- dispatch
template <typename T, int VW>
struct LnDispatch {
  template <int NV>
  static void fwd(int grid, T* y, T* mu, T* rs, const T* x, const T* w, const T* b, int64_t rows, int cols, T eps) {
    ln_fwd_kernel<T, NV, VW><<<grid, 256, 0, stream()>>>(y, mu, rs, x, w, b, rows, cols, eps);
  }
  template <int NV>
  static void bwd(int grid, T* dx, T* pdw, T* pdb, const T* dy, const T* x, const T* w, const T* mu, const T* rs,
                  const T* add, int64_t rows, int cols, int acc) {
    size_t lds = (size_t)4 * 2 * NV * VW * 64 * sizeof(T);
    ln_bwd_kernel<T, NV, VW><<<grid, 256, lds, stream()>>>(dx, pdw, pdb, dy, x, w, mu, rs, add, rows, cols, acc);
  }
  // dy as two split-K partials (rows of up to 8 vectors per lane) or four
  // (up to 4 vectors per lane)
  template <int NV>
  static void bwd2(int grid, int np, T* dx, T* pdw, T* pdb, const T* dy, int64_t pstride, const T* x, const T* w,
                   const T* mu, const T* rs, const T* add, int64_t rows, int cols, int acc) {
    size_t lds = (size_t)4 * 2 * NV * VW * 64 * sizeof(T);
    if constexpr (NV <= 4) {
      if (np == 4) {
        ln_bwd_kernel<T, NV, VW, 4><<<grid, 256, lds, stream()>>>(dx, pdw, pdb, dy, x, w, mu, rs, add, rows, cols,
                                                                 acc, pstride);
        return;
      }
    }
    if constexpr (NV <= 8) {
      ln_bwd_kernel<T, NV, VW, 2><<<grid, 256, lds, stream()>>>(dx, pdw, pdb, dy, x, w, mu, rs, add, rows, cols, acc,
                                                               pstride);
    }
  }
};

template <typename T>
static int ln_fwd(void* y, void* mean, void* rstd, const void* x, const void* w, const void* b, int64_t rows,
                  int64_t cols, double eps) {
  constexpr int VWV = 16 / sizeof(T);
  bool vec = cols % VWV == 0 && aligned(x, 16) && aligned(y, 16) && aligned(w, 16) && aligned(b, 16);
  int vw = vec ? VWV : 1;
  int nv = ln_pick_nv(cdiv(cols, 64LL * vw));
  if (nv < 0) {  // longer rows than a wave holds
    TimedLaunch tl(DTMI_FAM_OTHER, (double)rows * cols * 2 * sizeof(T));
    const unsigned g = (unsigned)(rows < 4096 ? rows : 4096);
    ln_fwd_wide_kernel<T><<<g, 256, 0, stream()>>>((T*)y, (T*)mean, (T*)rstd, (const T*)x, (const T*)w,
                                                    (const T*)b, rows, cols, (T)eps);
    LAUNCH_CHECK("ln_fwd_wide_kernel");
    return DTMI_OK;
  }
  int grid = (int)cdiv(rows, 4);
  TimedLaunch tl(DTMI_FAM_OTHER, (double)rows * cols * 2 * sizeof(T));
  T* Y = (T*)y;
  T* MU = (T*)mean;
  T* RS = (T*)rstd;
  const T *X = (const T*)x, *W = (const T*)w, *B = (const T*)b;
  int c = (int)cols;
  T e = (T)eps;
  if (vec) {
#define CALLV(NV) LnDispatch<T, VWV>::template fwd<NV>(grid, Y, MU, RS, X, W, B, rows, c, e)
    LN_NV_SWITCH(nv, CALLV)
#undef CALLV
  } else {
#define CALLS(NV) LnDispatch<T, 1>::template fwd<NV>(grid, Y, MU, RS, X, W, B, rows, c, e)
    LN_NV_SWITCH(nv, CALLS)
#undef CALLS
  }
  LAUNCH_CHECK("ln_fwd_kernel");
  return DTMI_OK;
}

template <typename T>
static int ln_bwd(void* dx, void* dw, void* db, const void* dy, const void* x, const void* w, const void* mean,
                  const void* rstd, const void* addend, int64_t rows, int64_t cols, int accumulate,
                  void* scratch_ptr = nullptr, size_t scratch_bytes = 0, int nparts = 1) {
  constexpr int VWV = 16 / sizeof(T);
  bool vec = cols % VWV == 0 && aligned(x, 16) && aligned(dy, 16) && aligned(dx, 16) && aligned(w, 16) &&
             aligned(addend, 16);
  int vw = vec ? VWV : 1;
  const int nv = ln_pick_nv(cdiv(cols, 64LL * vw));
  const bool wide = nv < 0;  // longer rows than a wave holds
  if (nparts > 1) {
    // dy as split-K partials: summed in the kernel's loads (two partials on
    // aligned rows of up to 8 vectors per lane, four on rows of up to 4),
    // else by a sum pass first
    const int64_t pstride = rows * cols;
    if (((nparts == 2 && nv <= 8) || (nparts == 4 && nv <= 4)) && vec && nv > 0 &&
        (pstride * (int64_t)sizeof(T)) % 16 == 0) {
      const int grid = ln_bwd_blocks(rows);
      void* parts = nullptr;
      int rc = pool_alloc(&parts, (size_t)2 * grid * cols * sizeof(T));
      if (rc) return rc;
      T* pdw = (T*)parts;
      T* pdb = pdw + (size_t)grid * cols;
      {
        const double arrays = nparts + ((addend || (accumulate & 1)) ? 3.0 : 2.0);
        TimedLaunch tl(DTMI_FAM_LN_BWD, (double)rows * cols * arrays * sizeof(T));
        const int c = (int)cols;
        const int acc = (accumulate & 1) ? 1 : 0;
#define CALLP(NV)                                                                                        \
  LnDispatch<T, VWV>::template bwd2<NV>(grid, nparts, (T*)dx, pdw, pdb, (const T*)dy, pstride, (const T*)x,      \
                                        (const T*)w, (const T*)mean, (const T*)rstd, (const T*)addend, rows, c, acc)
        LN_NV_SWITCH(nv, CALLP)
#undef CALLP
        launch_colreduce<T>((T*)dw, pdw, grid, cols, (accumulate & 2) ? 1 : 0, (T*)db, pdb);
      }
      hipError_t le = hipGetLastError();
      pool_free(parts);
      if (le != hipSuccess) return fail_hip(le, "ln_bwd kernels", __FILE__, __LINE__);
      return DTMI_OK;
    }
    void* sum = nullptr;
    int rc = pool_alloc(&sum, (size_t)pstride * sizeof(T));
    if (rc) return rc;
    const int64_t g = cdiv(pstride, 256LL) < 8192 ? cdiv(pstride, 256LL) : 8192;
    sum_parts_kernel<T><<<(unsigned)g, 256, 0, stream()>>>((T*)sum, (const T*)dy, pstride, nparts);
    rc = ln_bwd<T>(dx, dw, db, sum, x, w, mean, rstd, addend, rows, cols, accumulate);
    pool_free(sum);
    return rc;
  }
  const int grid = wide ? ln_bwd_wide_blocks(rows, cols, sizeof(T)) : ln_bwd_blocks(rows);
  const size_t part_bytes = (size_t)2 * grid * cols * sizeof(T);
  void* parts = scratch_ptr;
  if (scratch_ptr) {
    DTMI_CHECK(part_bytes <= scratch_bytes,
               "dtmi_layernorm_bwd_noalloc: [%lld, %lld] needs %zu bytes of column partials, more than the %zu "
               "of its scratch array (use dtmi_layernorm_bwd)",
               (long long)rows, (long long)cols, part_bytes, scratch_bytes);
  } else {
    int rc = pool_alloc(&parts, part_bytes);
    if (rc) return rc;
  }
  T* pdw = (T*)parts;
  T* pdb = pdw + (size_t)grid * cols;
  {
    // x and dy in, dx out, and the addend (or the existing dx) in when summed
    const double arrays = (addend || (accumulate & 1)) ? 4.0 : 3.0;
    // the allocation-free form is not timed: timing creates HIP events
    TimedLaunch tl(scratch_ptr ? -1 : DTMI_FAM_LN_BWD, (double)rows * cols * arrays * sizeof(T));
    T* DX = (T*)dx;
    const T *DY = (const T*)dy, *X = (const T*)x, *W = (const T*)w, *MU = (const T*)mean, *RS = (const T*)rstd;
    int c = (int)cols;
    int acc = (accumulate & 1) ? 1 : 0;
    const T* ADD = (const T*)addend;
    if (wide) {
      ln_bwd_wide_kernel<T><<<grid, 256, 0, stream()>>>(DX, pdw, pdb, DY, X, W, MU, RS, ADD, rows, cols, acc);
    } else if (vec) {
#define CALLV(NV) LnDispatch<T, VWV>::template bwd<NV>(grid, DX, pdw, pdb, DY, X, W, MU, RS, ADD, rows, c, acc)
      LN_NV_SWITCH(nv, CALLV)
#undef CALLV
    } else {
#define CALLS(NV) LnDispatch<T, 1>::template bwd<NV>(grid, DX, pdw, pdb, DY, X, W, MU, RS, ADD, rows, c, acc)
      LN_NV_SWITCH(nv, CALLS)
#undef CALLS
    }
    launch_colreduce<T>((T*)dw, pdw, grid, cols, (accumulate & 2) ? 1 : 0, (T*)db, pdb);
  }
  hipError_t le = hipGetLastError();
  if (!scratch_ptr) pool_free(parts);
  if (le != hipSuccess) return fail_hip(le, "ln_bwd kernels", __FILE__, __LINE__);
  return DTMI_OK;
}

// -------------------------------------------- allocation-free entry point
// The dgamma / dbeta column partials of dtmi_layernorm_bwd_noalloc live in a
// file-scope device array: every GPU the library runs on holds its own copy
// until the process ends. In host code `scratch` names only a host-side
// stand-in, so the address each device's copy has is taken once per device
// with hipGetSymbolAddress (dtmi_init, with the device current) and only that
// address is handed to kernels.
constexpr size_t kLnScratchBytes = (size_t)8 << 20;
static __device__ __align__(256) unsigned char scratch[kLnScratchBytes];
constexpr int kMaxDevices = 64;
static void* g_scratch_ptr[kMaxDevices];

int ln_scratch_setup(int device) {
  DTMI_CHECK(device >= 0 && device < kMaxDevices, "dtmi_init: device %d beyond %d", device, kMaxDevices);
  if (g_scratch_ptr[device]) return DTMI_OK;
  void* p = nullptr;
  hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return fail_hip(e, "hipGetSymbolAddress(scratch)", __FILE__, __LINE__);
  DTMI_CHECK(p != nullptr, "dtmi_init: no device address for the LayerNorm scratch array");
  g_scratch_ptr[device] = p;
  return DTMI_OK;
}

}  // namespace dtmi

using namespace dtmi;

DTMI_EXPORT int dtmi_layernorm_fwd(int dtype, void* y, void* mean, void* rstd, const void* x, const void* w,
                                   const void* b, int64_t rows, int64_t cols, double eps) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_DTYPE_OK(dtype);
  DTMI_CHECK(rows >= 0 && cols > 0 && cols < (1 << 30), "dtmi_layernorm_fwd: bad shape [%lld, %lld]", (long long)rows,
             (long long)cols);
  if (rows == 0) return DTMI_OK;
  DTMI_CHECK(y && mean && rstd && x && w && b, "dtmi_layernorm_fwd: NULL pointer");
  if (dtype == DTMI_F32) return ln_fwd<float>(y, mean, rstd, x, w, b, rows, cols, eps);
  return ln_fwd<double>(y, mean, rstd, x, w, b, rows, cols, eps);
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_layernorm_bwd(int dtype, void* dx, void* dw, void* db, const void* dy, const void* x,
                                   const void* w, const void* mean, const void* rstd, int64_t rows, int64_t cols,
                                   int accumulate) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_DTYPE_OK(dtype);
  DTMI_CHECK(rows >= 0 && cols > 0 && cols < (1 << 30), "dtmi_layernorm_bwd: bad shape [%lld, %lld]", (long long)rows,
             (long long)cols);
  DTMI_CHECK(dw && db, "dtmi_layernorm_bwd: NULL dgamma/dbeta");
  if (rows == 0) {
    if (accumulate & 2) return DTMI_OK;
    int rc = dtmi_fill(dtype, dw, 0.0, cols);
    return rc ? rc : dtmi_fill(dtype, db, 0.0, cols);
  }
  DTMI_CHECK(dx && dy && x && w && mean && rstd, "dtmi_layernorm_bwd: NULL pointer");
  if (dtype == DTMI_F32) return ln_bwd<float>(dx, dw, db, dy, x, w, mean, rstd, nullptr, rows, cols, accumulate);
  return ln_bwd<double>(dx, dw, db, dy, x, w, mean, rstd, nullptr, rows, cols, accumulate);
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_layernorm_bwd_parts(int dtype, void* dx, void* dw, void* db, const void* dy_parts, int nparts,
                                         const void* x, const void* w, const void* mean, const void* rstd,
                                         const void* dx_addend, int64_t rows, int64_t cols, int accumulate) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_DTYPE_OK(dtype);
  DTMI_CHECK(rows >= 0 && cols > 0 && cols < (1 << 30) && nparts >= 1 && nparts <= 64,
             "dtmi_layernorm_bwd_parts: bad shape [%lld, %lld] or part count %d", (long long)rows, (long long)cols,
             nparts);
  DTMI_CHECK(dw && db, "dtmi_layernorm_bwd_parts: NULL dgamma/dbeta");
  DTMI_CHECK(!(dx_addend && (accumulate & 1)), "dtmi_layernorm_bwd_parts: an addend and accumulate bit 0 together");
  if (rows == 0) {
    if (accumulate & 2) return DTMI_OK;
    int rc = dtmi_fill(dtype, dw, 0.0, cols);
    return rc ? rc : dtmi_fill(dtype, db, 0.0, cols);
  }
  DTMI_CHECK(dx && dy_parts && x && w && mean && rstd, "dtmi_layernorm_bwd_parts: NULL pointer");
  {
    // dx is written while other waves still read rows of the partials and
    // the addend: the byte ranges must be disjoint
    const size_t bytes = (size_t)rows * (size_t)cols * (dtype == DTMI_F32 ? 4 : 8);
    const uintptr_t d0 = (uintptr_t)dx, p0 = (uintptr_t)dy_parts;
    DTMI_CHECK(p0 + bytes * (size_t)nparts <= d0 || d0 + bytes <= p0,
               "dtmi_layernorm_bwd_parts: the partials overlap dx");
    if (dx_addend) {
      const uintptr_t a0 = (uintptr_t)dx_addend;
      DTMI_CHECK(a0 + bytes <= d0 || d0 + bytes <= a0, "dtmi_layernorm_bwd_parts: the addend overlaps dx");
    }
  }
  if (dtype == DTMI_F32)
    return ln_bwd<float>(dx, dw, db, dy_parts, x, w, mean, rstd, dx_addend, rows, cols, accumulate, nullptr, 0,
                         nparts);
  return ln_bwd<double>(dx, dw, db, dy_parts, x, w, mean, rstd, dx_addend, rows, cols, accumulate, nullptr, 0, nparts);
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_layernorm_bwd_add(int dtype, void* dx, void* dw, void* db, const void* dy, const void* x,
                                       const void* w, const void* mean, const void* rstd, const void* dx_addend,
                                       int64_t rows, int64_t cols, int accumulate) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_DTYPE_OK(dtype);
  DTMI_CHECK(rows >= 0 && cols > 0 && cols < (1 << 30), "dtmi_layernorm_bwd_add: bad shape [%lld, %lld]",
             (long long)rows, (long long)cols);
  DTMI_CHECK(dw && db, "dtmi_layernorm_bwd_add: NULL dgamma/dbeta");
  DTMI_CHECK(!(accumulate & 1), "dtmi_layernorm_bwd_add: dx takes the addend, not accumulate bit 0");
  if (rows == 0) {
    if (accumulate & 2) return DTMI_OK;
    int rc = dtmi_fill(dtype, dw, 0.0, cols);
    return rc ? rc : dtmi_fill(dtype, db, 0.0, cols);
  }
  DTMI_CHECK(dx && dy && x && w && mean && rstd && dx_addend, "dtmi_layernorm_bwd_add: NULL pointer");
  {
    // dx is written while other waves still read rows of the addend: the two
    // byte ranges must be disjoint (an exact alias is what accumulate bit 0 does)
    const size_t bytes = (size_t)rows * (size_t)cols * (dtype == DTMI_F32 ? 4 : 8);
    const uintptr_t a0 = (uintptr_t)dx_addend, d0 = (uintptr_t)dx;
    DTMI_CHECK(a0 + bytes <= d0 || d0 + bytes <= a0,
               "dtmi_layernorm_bwd_add: the addend overlaps dx (for dx += use accumulate bit 0 instead)");
  }
  if (dtype == DTMI_F32)
    return ln_bwd<float>(dx, dw, db, dy, x, w, mean, rstd, dx_addend, rows, cols, accumulate);
  return ln_bwd<double>(dx, dw, db, dy, x, w, mean, rstd, dx_addend, rows, cols, accumulate);
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_layernorm_bwd_noalloc(int dtype, void* dx, void* dw, void* db, const void* dy, const void* x,
                                           const void* w, const void* mean, const void* rstd, int64_t rows,
                                           int64_t cols, int accumulate) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_DTYPE_OK(dtype);
  DTMI_CHECK(rows >= 0 && cols > 0 && cols < (1 << 30), "dtmi_layernorm_bwd_noalloc: bad shape [%lld, %lld]",
             (long long)rows, (long long)cols);
  DTMI_CHECK(dw && db, "dtmi_layernorm_bwd_noalloc: NULL dgamma/dbeta");
  if (rows == 0) {
    if (accumulate & 2) return DTMI_OK;
    int rc = dtmi_fill(dtype, dw, 0.0, cols);
    return rc ? rc : dtmi_fill(dtype, db, 0.0, cols);
  }
  DTMI_CHECK(dx && dy && x && w && mean && rstd, "dtmi_layernorm_bwd_noalloc: NULL pointer");
  const int dev = device_id();
  void* sp = dev >= 0 && dev < kMaxDevices ? g_scratch_ptr[dev] : nullptr;
  DTMI_CHECK(sp != nullptr, "dtmi_layernorm_bwd_noalloc: scratch array not set up on device %d", dev);
  if (dtype == DTMI_F32)
    return ln_bwd<float>(dx, dw, db, dy, x, w, mean, rstd, nullptr, rows, cols, accumulate, sp, kLnScratchBytes);
  return ln_bwd<double>(dx, dw, db, dy, x, w, mean, rstd, nullptr, rows, cols, accumulate, sp, kLnScratchBytes);
  DTMI_BODY_END
}
