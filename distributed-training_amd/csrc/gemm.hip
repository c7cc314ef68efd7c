// Dense contractions on the MFMA matrix cores: C = sum_k A(m,k) B(k,n) (+ bias)
// in float32 (v_mfma_f32_32x32x2_f32) and float64 (v_mfma_f64_16x16x4_f64).
//
// Behind dtrain's matmul node (dtrain/autograd.py:102-109) and Linear
// (dtrain/nn.py:58-65): forward Y = X W (+ b), dX = dY W^T, dW = X^T dY.
// Row-major operands in either orientation:
//   A "KC": A(m,k) = A[m*lda + k]  (X, dY)      A "MC": A(m,k) = A[k*lda + m]  (X^T)
//   B "NC": B(k,n) = B[k*ldb + n]  (W, dY)      B "KC": B(k,n) = B[n*ldb + k]  (W^T)
//
// Tiling. 256 threads = 4 waves in a 2x2 grid; block tile 128x128; k-tile
// 16 floats or 8 doubles; MFMA tiles of 32x32 (float32) or 16x16 (float64).
// Each operand tile is staged in LDS in its global orientation (global -> LDS
// is a straight 16-byte vector copy, fully coalesced along the contiguous
// dimension), with one barrier per k-tile and the next tiles' global loads in
// flight during the MFMAs. The loads go through per-thread pointers set up
// once and advanced by one k-tile per load (rows past the matrix edge clamped
// onto the last row), so the main loop has no index arithmetic and no
// divergent branches; only a partial last k-tile is masked.
//   gemm_dma_kernel (16-byte aligned operands -- every GPT-2 GEMM, in float32
//     and float64): the loads go straight into LDS (global_load_lds_dwordx4)
//     through three stages, in swizzled layouts that keep the fragment reads
//     conflict-free.
//   gemm_kernel (unaligned operands): registers -> LDS, double-buffered.
//   gemm_x6_kernel (float32 when dtmi_set_gemm_math selects the split-bf16
//     arithmetic, aligned operands): each operand split exactly into three
//     bf16 parts on the way into LDS, six partial products on the bf16 MFMA
//     (its own section below).
// (256x128 and 128x256 tiles, 32-wide k-tiles, a two-tile register prefetch
// and AGPR accumulators measured no faster on the GPT-2 shapes.)
//
// MFMA k-slots. An MFMA takes k in lane groups g = lane / MT (2 groups of 32
// lanes for 32x32x2, 4 groups of 16 for 16x16x4). Within each 8-wide k chunk,
// step s of group g uses k = chunk + VEC*g + s (VEC = 4 floats or 2 doubles),
// the same permutation for A and B (a permutation of the reduction index does
// not change the sum's terms). With it a k-contiguous LDS tile gives a lane
// its VEC k-values with one 16-byte ds_read, and an mn-contiguous LDS tile is
// read with conflict-free 4/8-byte reads (row pads chosen so the lane groups
// fall in different LDS banks).
//
// Grid. Tiles are enumerated group-of-8-rows first (L2 reuse of B panels) and
// the linear block index is remapped so each of the 8 XCDs (blocks are dealt
// to XCDs round-robin) works on a contiguous range of tiles and shares its L2.
// Small tile counts with long K are split along K; the split partials are
// summed in split order by a second kernel (deterministic, no atomics).
#include "common.h"
#include "bufrsrc.h"
#include "gelu.h"
#include "rowln.h"

namespace dtmi {

template <typename T>
struct MF;

template <>
struct MF<float> {
  static constexpr int MT = 32, G = 2, VEC = 4, NACC = 16;
  typedef float acc_t __attribute__((ext_vector_type(16)));
  typedef float vec_t __attribute__((ext_vector_type(4)));
  static __device__ __forceinline__ acc_t mma(float a, float b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
  // result register i of lane group g holds row (8*(i/4) + 4*g + i%4), column lane%32
  static __device__ __forceinline__ int row(int i, int g) { return 8 * (i / 4) + 4 * g + (i % 4); }
};

template <>
struct MF<double> {
  static constexpr int MT = 16, G = 4, VEC = 2, NACC = 4;
  typedef double acc_t __attribute__((ext_vector_type(4)));
  typedef double vec_t __attribute__((ext_vector_type(2)));
  static __device__ __forceinline__ acc_t mma(double a, double b, acc_t c) {
    return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
  }
  // result register i of lane group g holds row (g + 4*i), column lane%16
  static __device__ __forceinline__ int row(int i, int g) { return g + 4 * i; }
};

struct GemmArgs {
  const void* A;
  const void* B;
  void* C;
  const void* bias;
  void* ws;  // split-K partials [splits][batch][M][N] (NULL when not split)
  int64_t M, N, K, lda, ldb, ldc;
  int64_t sA, sB, sC;  // batch strides (elements)
  int64_t k_per_split;
  int tiles_m, tiles_n;
  int accumulate;
  // Epilogue fusions (applied after the bias, in this order):
  const void* addend;  // residual: v = addend[m, n] + v   (row stride ldc)
  int epi;             // kEpiGeluFwd: aux = gelu(v), C keeps v; kEpiGeluBwd: C = gelu'(aux) * v
  void* aux;           // [M, N] with row stride ldc
  // Column sums of B over k (the bias gradient of dW = X^T dY: db = sum over
  // rows of dY), taken by the blocks of the first row of tiles from the B
  // tiles already in LDS. Unbatched only. With split-K each split's sums go to
  // colsum_ws[split][n] and the reduction kernel adds them in split order.
  void* colsum;
  void* colsum_ws;
  int colsum_accumulate;
};

constexpr int kEpiNone = 0, kEpiGeluFwd = 1, kEpiGeluBwd = 2;

// The fused epilogue of one output element v (the k-sum of row m, column n):
// bias, residual, accumulate, GELU -- the operation order of the unfused
// graph (Linear adds its bias, then the residual add, then GELU / its
// backward as dtrain/autograd.py:133-144 computes them).
template <typename T>
__device__ __forceinline__ void epilogue_store(const GemmArgs& a, T* __restrict__ C, int64_t ldc, int64_t m,
                                               int64_t n, T v, int64_t batch) {
  if (a.bias) v = v + ((const T*)a.bias)[n];
  const int64_t o = m * ldc + n;
  if (a.addend) v = ((const T*)a.addend)[batch * a.sC + o] + v;
  if (a.accumulate) v = C[o] + v;
  if (a.epi == kEpiGeluFwd) {
    ((T*)a.aux)[batch * a.sC + o] = gelu_f<T>(v);
  } else if (a.epi == kEpiGeluBwd) {
    v = gelu_b<T>(((const T*)a.aux)[batch * a.sC + o], v);
  }
  C[o] = v;
}

constexpr int kKC = 8;
// k-tile: 16 floats or 8 doubles
template <typename T>
constexpr int kBKT = sizeof(T) == 4 ? 16 : 8;

// One operand tile of BMN rows/columns (along M or N) by kBK.
template <typename T, bool KCONTIG, int BMN>
struct TileLayout {
  static constexpr int VEC = MF<T>::VEC;
  static constexpr int kBK = kBKT<T>;
  // k-contiguous: [mn][kBK + VEC]; mn-contiguous: [kBK][BMN + 8]
  static constexpr int STRIDE = KCONTIG ? (kBK + VEC) : (BMN + 8);
  static constexpr int SIZE = KCONTIG ? BMN * STRIDE : kBK * STRIDE;
  static constexpr int NVEC = BMN * kBK / VEC / 256;  // 16-byte vectors per thread per tile
};

template <typename T, bool KCONTIG, int BMN>
struct TileRegs {
  typename MF<T>::vec_t v[TileLayout<T, KCONTIG, BMN>::NVEC];
};

// Global -> registers for one BMN x kBK operand tile (mn0 = first row/col of
// the tile along M or N, k0 = first k). Out-of-range elements read as 0.
template <typename T, bool KCONTIG, int BMN, bool VECLD>
__device__ __forceinline__ void load_tile(TileRegs<T, KCONTIG, BMN>& r, const T* __restrict__ P, int64_t ld,
                                          int64_t mn0, int64_t MN, int64_t k0, int64_t kend) {
  using L = TileLayout<T, KCONTIG, BMN>;
  constexpr int VEC = L::VEC;
  constexpr int kBK = L::kBK;
#pragma unroll
  for (int i = 0; i < L::NVEC; ++i) {
    const int f = threadIdx.x + 256 * i;
    int64_t mn, k;
    if (KCONTIG) {
      mn = mn0 + f / (kBK / VEC);
      k = k0 + (f % (kBK / VEC)) * VEC;
    } else {
      k = k0 + f / (BMN / VEC);
      mn = mn0 + (f % (BMN / VEC)) * VEC;
    }
    if (VECLD) {
      // every dimension that vectors run along is a multiple of VEC
      if (mn < MN && k < kend) {
        const T* src = KCONTIG ? P + mn * ld + k : P + k * ld + mn;
        r.v[i] = *reinterpret_cast<const typename MF<T>::vec_t*>(src);
      } else {
        r.v[i] = typename MF<T>::vec_t(0);
      }
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        int64_t mm = KCONTIG ? mn : mn + e;
        int64_t kk = KCONTIG ? k + e : k;
        r.v[i][e] = (mm < MN && kk < kend) ? (KCONTIG ? P[mm * ld + kk] : P[kk * ld + mm]) : T(0);
      }
    }
  }
}

// Per-thread source pointers for the vector loads of the k-tiles that lie
// wholly inside [kbeg, kend): set up once, advanced by one k-tile per load,
// so the main loop carries no index arithmetic and no bounds branches. Rows
// (or columns) past the matrix edge are clamped onto its last row/column:
// they feed only output rows/columns that the epilogue never stores.
template <typename T, bool KCONTIG, int BMN>
struct TilePtr {
  const T* p[TileLayout<T, KCONTIG, BMN>::NVEC];
  int64_t step;
};

template <typename T, bool KCONTIG, int BMN>
__device__ __forceinline__ void init_ptr(TilePtr<T, KCONTIG, BMN>& t, const T* __restrict__ P, int64_t ld,
                                         int64_t mn0, int64_t MN, int64_t kbeg) {
  using L = TileLayout<T, KCONTIG, BMN>;
  constexpr int VEC = L::VEC;
  constexpr int kBK = L::kBK;
#pragma unroll
  for (int i = 0; i < L::NVEC; ++i) {
    const int f = threadIdx.x + 256 * i;
    if (KCONTIG) {
      int64_t mn = mn0 + f / (kBK / VEC);
      mn = mn < MN ? mn : MN - 1;
      t.p[i] = P + mn * ld + kbeg + (f % (kBK / VEC)) * VEC;
    } else {
      int64_t mn = mn0 + (f % (BMN / VEC)) * VEC;
      mn = mn < MN ? mn : MN - VEC;
      t.p[i] = P + (kbeg + f / (BMN / VEC)) * ld + mn;
    }
  }
  t.step = KCONTIG ? (int64_t)kBK : (int64_t)kBK * ld;
}

template <typename T, bool KCONTIG, int BMN>
__device__ __forceinline__ void load_fast(TileRegs<T, KCONTIG, BMN>& r, TilePtr<T, KCONTIG, BMN>& t) {
#pragma unroll
  for (int i = 0; i < TileLayout<T, KCONTIG, BMN>::NVEC; ++i) {
    r.v[i] = *reinterpret_cast<const typename MF<T>::vec_t*>(t.p[i]);
    t.p[i] += t.step;
  }
}

// The last k-tile when it extends past kend: the same number of loads as a
// full tile, from addresses clamped into [kbeg, kend) (k past kend is zeroed
// when the tile is stored to LDS, see store_tile_masked).
template <typename T, bool KCONTIG, int BMN>
__device__ __forceinline__ void load_tail(TileRegs<T, KCONTIG, BMN>& r, const TilePtr<T, KCONTIG, BMN>& t,
                                          int64_t ld, int64_t k0, int64_t kend) {
  using L = TileLayout<T, KCONTIG, BMN>;
  constexpr int VEC = L::VEC;
  constexpr int kBK = L::kBK;
#pragma unroll
  for (int i = 0; i < L::NVEC; ++i) {
    const int f = threadIdx.x + 256 * i;
    const T* q;
    if (KCONTIG) {
      const int64_t k = k0 + (f % (kBK / VEC)) * VEC;
      q = t.p[i] - (k < kend ? 0 : k - (kend - VEC));
    } else {
      const int64_t k = k0 + f / (BMN / VEC);
      q = t.p[i] - (k < kend ? 0 : (k - (kend - 1)) * ld);
    }
    r.v[i] = *reinterpret_cast<const typename MF<T>::vec_t*>(q);
  }
}

template <typename T, bool KCONTIG, int BMN>
__device__ __forceinline__ void store_tile(T* __restrict__ lds, const TileRegs<T, KCONTIG, BMN>& r) {
  using L = TileLayout<T, KCONTIG, BMN>;
  constexpr int VEC = L::VEC;
  constexpr int kBK = L::kBK;
#pragma unroll
  for (int i = 0; i < L::NVEC; ++i) {
    const int f = threadIdx.x + 256 * i;
    int off;
    if (KCONTIG)
      off = (f / (kBK / VEC)) * L::STRIDE + (f % (kBK / VEC)) * VEC;
    else
      off = (f / (BMN / VEC)) * L::STRIDE + (f % (BMN / VEC)) * VEC;
    *reinterpret_cast<typename MF<T>::vec_t*>(lds + off) = r.v[i];
  }
}

// store_tile for the last, partial k-tile: vectors whose k is at or past
// kend are stored as zeros.
template <typename T, bool KCONTIG, int BMN>
__device__ __forceinline__ void store_tile_masked(T* __restrict__ lds, const TileRegs<T, KCONTIG, BMN>& r,
                                                  int64_t k0, int64_t kend) {
  using L = TileLayout<T, KCONTIG, BMN>;
  constexpr int VEC = L::VEC;
  constexpr int kBK = L::kBK;
#pragma unroll
  for (int i = 0; i < L::NVEC; ++i) {
    const int f = threadIdx.x + 256 * i;
    int off;
    int64_t k;
    if (KCONTIG) {
      off = (f / (kBK / VEC)) * L::STRIDE + (f % (kBK / VEC)) * VEC;
      k = k0 + (f % (kBK / VEC)) * VEC;
    } else {
      off = (f / (BMN / VEC)) * L::STRIDE + (f % (BMN / VEC)) * VEC;
      k = k0 + f / (BMN / VEC);
    }
    *reinterpret_cast<typename MF<T>::vec_t*>(lds + off) = k < kend ? r.v[i] : typename MF<T>::vec_t(0);
  }
}

// The VEC k-values lane (group g, position c) feeds for operand rows/cols
// `base + c` at chunk `kk`.
template <typename T, bool KCONTIG, int BMN>
__device__ __forceinline__ typename MF<T>::vec_t read_frag(const T* __restrict__ lds, int base, int kk, int g, int c) {
  using L = TileLayout<T, KCONTIG, BMN>;
  constexpr int VEC = L::VEC;
  typename MF<T>::vec_t v;
  if (KCONTIG) {
    v = *reinterpret_cast<const typename MF<T>::vec_t*>(lds + (base + c) * L::STRIDE + kk + VEC * g);
  } else {
#pragma unroll
    for (int s = 0; s < VEC; ++s) v[s] = lds[(kk + VEC * g + s) * L::STRIDE + base + c];
  }
  return v;
}

__device__ __forceinline__ void tile_coords_of(const GemmArgs& a, int t, int& tm, int& tn) {
  const int nt = a.tiles_m * a.tiles_n;
  if ((nt & 7) == 0) t = (t & 7) * (nt >> 3) + (t >> 3);  // contiguous tile range per XCD
  constexpr int GROUP = 8;
  const int per_group = GROUP * a.tiles_n;
  const int group = t / per_group;
  const int first_m = group * GROUP;
  const int gsz = a.tiles_m - first_m < GROUP ? a.tiles_m - first_m : GROUP;
  const int r = t - group * per_group;
  tm = first_m + r % gsz;
  tn = r / gsz;
}
__device__ __forceinline__ void tile_coords(const GemmArgs& a, int& tm, int& tn) {
  tile_coords_of(a, (int)blockIdx.x, tm, tn);
}

// The column sum of one B column over this block's k range: to colsum (or
// added to it), or, with split-K, to the split's row of colsum_ws.
template <typename T>
__device__ __forceinline__ void finish_colsum(const GemmArgs& a, double csum, int64_t n, int split) {
  if (n >= a.N) return;
  if (a.colsum_ws) {
    ((T*)a.colsum_ws)[(int64_t)split * a.N + n] = (T)csum;
  } else {
    T* cs = (T*)a.colsum;
    cs[n] = a.colsum_accumulate ? cs[n] + (T)csum : (T)csum;
  }
}

// A wave's TM x TN MFMA accumulators (its tile starts at row m0, column n0):
// split-K partials go to the workspace as they are; otherwise the fused
// epilogue writes C (and aux).
template <typename T, int TM, int TN, bool FAST_EPI = false>
__device__ __forceinline__ void write_acc(const GemmArgs& a, const typename MF<T>::acc_t (&acc)[TM][TN], int64_t m0,
                                          int64_t n0, int g, int c, int split, int64_t batch) {
  using MFT = MF<T>;
  constexpr int MT = MFT::MT, NACC = MFT::NACC;
  const bool to_ws = a.ws != nullptr;
  T* C = to_ws ? (T*)a.ws + ((int64_t)split * gridDim.z + batch) * a.M * a.N : (T*)a.C + batch * a.sC;
  const int64_t ldc = to_ws ? a.N : a.ldc;
  if constexpr (FAST_EPI && std::is_same<T, float>::value) {
    if ((to_ws || (a.addend == nullptr && !a.accumulate)) && m0 + TM * MT <= a.M && n0 + TN * MT <= a.N) {
      // A whole wave tile in range with no residual or accumulation (every
      // split-K partial, the bias-only products, the GELU epilogues): buffer
      // accesses off the wave tile's corner -- one lane offset, and per
      // element a wave-uniform offset, so no per-element address arithmetic
      // on the SIMD the MFMAs share. The GELU backward's pre-activation of a
      // row of MFMA tiles is read before its first store (the stores may
      // alias it as far as the compiler can tell). Same operations as
      // epilogue_store.
      const int64_t corner = m0 * ldc + n0;
      const float* bias = to_ws ? nullptr : (const float*)a.bias;
      const Rsrc rc = make_rsrc(C + corner, ~0ull);
      const Rsrc rx = make_rsrc(to_ws ? C : (const float*)a.aux + batch * a.sC + corner, ~0ull);
      const uint32_t voff = (uint32_t)((4 * g * ldc + c) * 4);
      auto run = [&](auto modec) {
        constexpr int MODE = decltype(modec)::value;  // an epilogue kind
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          float x[TN][NACC];
          if constexpr (MODE == kEpiGeluBwd) {
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
              for (int r = 0; r < NACC; ++r)
                x[j][r] = buf_load1(rx, voff, (uint32_t)(((i * MT + MFT::row(r, 0)) * ldc + j * MT) * 4));
          }
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            const float bn = bias ? bias[n0 + j * MT + c] : 0.f;
#pragma unroll
            for (int r = 0; r < NACC; ++r) {
              const uint32_t so = (uint32_t)(((i * MT + MFT::row(r, 0)) * ldc + j * MT) * 4);
              float v = acc[i][j][r];
              if (bias) v = v + bn;
              if constexpr (MODE == kEpiGeluFwd) buf_store1(gelu_f<float>(v), rx, voff, so);
              if constexpr (MODE == kEpiGeluBwd) v = gelu_b<float>(x[j][r], v);
              buf_store1(v, rc, voff, so);
            }
          }
        }
      };
      const int epi = to_ws ? kEpiNone : a.epi;
      if (epi == kEpiGeluBwd)
        run(std::integral_constant<int, kEpiGeluBwd>());
      else if (epi == kEpiGeluFwd)
        run(std::integral_constant<int, kEpiGeluFwd>());
      else
        run(std::integral_constant<int, kEpiNone>());
      return;
    }
  }
  const bool plain = to_ws || (a.addend == nullptr && a.epi == kEpiNone && !a.accumulate);
  if (plain) {  // raw split-K partial, or v + bias
    const T* bias = to_ws ? nullptr : (const T*)a.bias;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int64_t n = n0 + j * MT + c;
        if (n >= a.N) continue;
        const T bn = bias ? bias[n] : T(0);
#pragma unroll
        for (int r = 0; r < NACC; ++r) {
          const int64_t m = m0 + i * MT + MFT::row(r, g);
          if (m >= a.M) continue;
          T v = acc[i][j][r];
          if (bias) v = v + bn;
          C[m * ldc + n] = v;
        }
      }
  } else {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int64_t n = n0 + j * MT + c;
        if (n >= a.N) continue;
#pragma unroll
        for (int r = 0; r < NACC; ++r) {
          const int64_t m = m0 + i * MT + MFT::row(r, g);
          if (m >= a.M) continue;
          epilogue_store<T>(a, C, ldc, m, n, acc[i][j][r], batch);
        }
      }
  }
}

// Block tile BM x BN, 4 waves in a 2 x 2 grid of (BM/2) x (BN/2) wave tiles.
template <typename T, int BM, int BN, bool AKC, bool BKC, bool VECA, bool VECB>
__global__ void __launch_bounds__(256, 2) gemm_kernel(GemmArgs a) {
  constexpr int kBK = kBKT<T>;
  using MFT = MF<T>;
  using LA = TileLayout<T, AKC, BM>;
  using LB = TileLayout<T, BKC, BN>;
  constexpr int MT = MFT::MT, VEC = MFT::VEC, NACC = MFT::NACC;
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int TM = WM / MT, TN = WN / MT;
  constexpr int NCH = kBK / kKC;  // 8-wide k chunks per k-tile
  __shared__ __attribute__((aligned(16))) T lds[2 * (LA::SIZE + LB::SIZE)];

  int tm, tn;
  tile_coords(a, tm, tn);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int split = blockIdx.y;
  const int64_t batch = blockIdx.z;
  const int64_t kbeg = (int64_t)split * a.k_per_split;
  const int64_t kend = kbeg + a.k_per_split < a.K ? kbeg + a.k_per_split : a.K;
  const T* A = (const T*)a.A + batch * a.sA;
  const T* B = (const T*)a.B + batch * a.sB;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane / MT, c = lane % MT;
  const int wm0 = (wave >> 1) * WM, wn0 = (wave & 1) * WN;

  typename MFT::acc_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = typename MFT::acc_t(0);

  // LDS is double-buffered with one barrier per k-tile: iteration kt issues
  // the global loads of tile kt+1 into registers, computes tile kt from LDS
  // stage kt&1 while they are in flight, then stores them to the other stage.
  TileRegs<T, AKC, BM> ra;
  TileRegs<T, BKC, BN> rb;
  const int64_t ntiles = kend > kbeg ? (kend - kbeg + kBK - 1) / kBK : 0;
  const int64_t nfull = kend > kbeg ? (kend - kbeg) / kBK : 0;  // tiles with every k in range
  TilePtr<T, AKC, BM> pa;
  TilePtr<T, BKC, BN> pb;
  if (VECA) init_ptr<T, AKC, BM>(pa, A, a.lda, m0, a.M, kbeg);
  if (VECB) init_ptr<T, BKC, BN>(pb, B, a.ldb, n0, a.N, kbeg);
  // Tiles are loaded strictly in order kt = 0, 1, 2, ...; only the last one
  // can be partial. Every tile issues the same loads with no divergent
  // branch and no index arithmetic beyond one pointer increment.
  auto load = [&](int64_t kt, TileRegs<T, AKC, BM>& la, TileRegs<T, BKC, BN>& lb) {
    const int64_t k0 = kbeg + kt * kBK;
    if (kt < nfull) {
      if (VECA) load_fast<T, AKC, BM>(la, pa);
      if (VECB) load_fast<T, BKC, BN>(lb, pb);
    } else {
      if (VECA) load_tail<T, AKC, BM>(la, pa, a.lda, k0, kend);
      if (VECB) load_tail<T, BKC, BN>(lb, pb, a.ldb, k0, kend);
    }
    if (!VECA) load_tile<T, AKC, BM, false>(la, A, a.lda, m0, a.M, k0, kend);
    if (!VECB) load_tile<T, BKC, BN, false>(lb, B, a.ldb, n0, a.N, k0, kend);
  };
  auto store = [&](int64_t kt, int stage, const TileRegs<T, AKC, BM>& sa, const TileRegs<T, BKC, BN>& sb) {
    T* As = lds + stage * LA::SIZE;
    T* Bs = lds + 2 * LA::SIZE + stage * LB::SIZE;
    if (kt < nfull) {
      store_tile<T, AKC, BM>(As, sa);
      store_tile<T, BKC, BN>(Bs, sb);
    } else {
      const int64_t k0 = kbeg + kt * kBK;
      store_tile_masked<T, AKC, BM>(As, sa, k0, kend);
      store_tile_masked<T, BKC, BN>(Bs, sb, k0, kend);
    }
  };
  if (ntiles > 0) {
    load(0, ra, rb);
    store(0, 0, ra, rb);
  }
  __syncthreads();
  const bool take_colsum = a.colsum != nullptr && tm == 0 && (int)threadIdx.x < BN;
  double csum = 0.0;
  for (int64_t kt = 0; kt < ntiles; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < ntiles) load(kt + 1, ra, rb);
    const T* As = lds + cur * LA::SIZE;
    const T* Bs = lds + 2 * LA::SIZE + cur * LB::SIZE;
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
      typename MFT::vec_t fa[TM], fb[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) fa[i] = read_frag<T, AKC, BM>(As, wm0 + i * MT, ch * kKC, g, c);
#pragma unroll
      for (int j = 0; j < TN; ++j) fb[j] = read_frag<T, BKC, BN>(Bs, wn0 + j * MT, ch * kKC, g, c);
#pragma unroll
      for (int s = 0; s < VEC; ++s)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] = MFT::mma(fa[i][s], fb[j][s], acc[i][j]);
    }
    if (take_colsum) {
      // this thread's column of the B tile: its kBK values in k order, then into
      // the running float64 sum (rows past kend were stored as zeros)
      T t = T(0);
#pragma unroll
      for (int k = 0; k < kBK; ++k) t = t + (BKC ? Bs[threadIdx.x * LB::STRIDE + k] : Bs[k * LB::STRIDE + threadIdx.x]);
      csum += (double)t;
    }
    if (kt + 1 < ntiles) store(kt + 1, cur ^ 1, ra, rb);
    __syncthreads();
  }
  if (take_colsum) finish_colsum<T>(a, csum, n0 + threadIdx.x, split);
  write_acc<T, TM, TN>(a, acc, m0 + wm0, n0 + wn0, g, c, split, batch);
}

// ---------------------------------------------------------------------------
// Direct global -> LDS loads (global_load_lds_dwordx4: each lane fetches 16
// bytes that land at LDS base + 16 * lane, with no register staging, no LDS
// store instructions and no wait before a store), float32 and float64 alike:
// a k-tile is 64 bytes of k per row (16 floats or 8 doubles), VEC = 16 bytes
// of elements (4 floats or 2 doubles) per vector. Three LDS stages: tile t's
// loads are issued two iterations before it is computed.
// LDS layouts (a 1 KB load instruction fills 1 KB contiguously, so conflicts
// are avoided by choosing which global vector each lane fetches):
//   KC  (k-contiguous operand, BMN rows x 64 bytes): 1 KB chunks of 16 rows;
//       the 16-byte k-vector v of chunk row r sits in 16-byte slot
//       4 r + (v ^ kc_swz(r)), so the 16-byte fragment reads of 16
//       consecutive rows hit distinct banks;
//   MNC (mn-contiguous operand, k-rows of BMN elements): k-row k holds its
//       mn-vectors u at slots u ^ mnc_swz(k), which flips 128 bytes between
//       the k-rows that the two lane groups of a half-wave fragment read
//       (k and k + 4 for float32, k and k + 2 for float64), so they hit
//       different bank halves.
constexpr int kDmaStages = 3;

__device__ __forceinline__ int kc_swz(int r) { return ((r >> 1) + (r >> 3)) & 3; }
template <typename T>
__device__ __forceinline__ int mnc_swz(int k) {
  return ((k >> (MF<T>::VEC == 4 ? 2 : 1)) & 1) << 3;
}

// Element offset, within one BMN x 64-byte operand tile, of the 16-byte
// vector of (row/col mn, k-vector v) for KC, or of (k-row k, mn-vector u)
// for MNC.
template <typename T>
__device__ __forceinline__ int kc_off(int mn, int v) {
  const int r = mn & 15;
  return (mn >> 4) * (1024 / (int)sizeof(T)) + (4 * r + (v ^ kc_swz(r))) * MF<T>::VEC;
}
template <typename T, int BMN>
__device__ __forceinline__ int mnc_off(int k, int u) {
  return k * BMN + (u ^ mnc_swz<T>(k)) * MF<T>::VEC;
}

// The BMN / 64 load instructions (1 KB each) of each wave per operand tile:
// a wave-uniform base address (the current k-tile's origin, advanced by
// scalar adds) and fixed per-lane 32-bit byte offsets, so issuing a tile
// takes no vector instructions. Offsets are >= 0: clamped rows / columns
// stay at or after the tile origin (the origin is inside the matrix, and
// MN - VEC >= mn0 because MN and mn0 are multiples of VEC).
template <typename T, bool KCONTIG, int BMN>
struct DmaSrc {
  static constexpr int NQ = BMN / 64;
  const T* base;
  unsigned off[NQ];
  int64_t step;  // elements per k-tile
};

template <typename T, bool KCONTIG, int BMN>
__device__ __forceinline__ void dma_init(DmaSrc<T, KCONTIG, BMN>& s, const T* __restrict__ P, int64_t ld,
                                         int64_t mn0, int64_t MN, int64_t kbeg, int wave, int lane) {
  constexpr int NQ = DmaSrc<T, KCONTIG, BMN>::NQ;
  constexpr int VEC = MF<T>::VEC;
  constexpr int RV = BMN / VEC;  // mn-vectors per k-row (MNC)
  s.base = KCONTIG ? P + mn0 * ld + kbeg : P + kbeg * ld + mn0;
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int j = wave * NQ + q;  // 1 KB chunk of the tile
    if (KCONTIG) {
      const int r = lane >> 2;
      int64_t mn = mn0 + 16 * j + r;
      mn = mn < MN ? mn : MN - 1;
      const int v = (lane & 3) ^ kc_swz(r);
      s.off[q] = (unsigned)(((mn - mn0) * ld + VEC * v) * (int64_t)sizeof(T));
    } else {
      const int k = (64 * j + lane) / RV;
      const int u = ((64 * j + lane) % RV) ^ mnc_swz<T>(k);
      int64_t mn = mn0 + VEC * u;
      mn = mn < MN ? mn : MN - VEC;
      s.off[q] = (unsigned)((k * ld + (mn - mn0)) * (int64_t)sizeof(T));
    }
  }
  s.step = KCONTIG ? 64 / (int)sizeof(T) : (64 / (int)sizeof(T)) * ld;
}

// Issue one operand tile: chunk q of this wave lands at LDS byte address
// lds_wave + LDS_OFF + 1024 q (lds_wave: wave-uniform, this wave's first
// chunk of stage 0). m0 takes the LDS address one wait state before the load.
// The asm writes no SCC (an s_add here would clobber the carry of a 64-bit
// scalar add the compiler may have split around it): the address is summed
// outside and moved in with s_mov_b32.
template <int LDS_OFF, typename T, bool KCONTIG, int BMN>
__device__ __forceinline__ void dma_issue(DmaSrc<T, KCONTIG, BMN>& s, unsigned lds_wave) {
  constexpr int NQ = DmaSrc<T, KCONTIG, BMN>::NQ;
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const unsigned dst = lds_wave + (unsigned)(LDS_OFF + 1024 * q);
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(s.off[q]), "s"(s.base),
                 "s"(dst)
                 : "memory", "m0");
  }
  s.base += s.step;
}

// This wave's loads except the newest N have landed, then every wave's have.
template <int N>
__device__ __forceinline__ void dma_wait_barrier() {
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
}

template <int V>
struct IC {
  static constexpr int value = V;
};

// The partial last k-tile through registers, stored in the same layouts
// (k at or past kend as zeros).
template <typename T, bool KCONTIG, int BMN>
__device__ __forceinline__ void dma_tail_store(T* __restrict__ tile, const TileRegs<T, KCONTIG, BMN>& r, int64_t k0,
                                               int64_t kend) {
  using L = TileLayout<T, KCONTIG, BMN>;
  constexpr int VEC = L::VEC;
  constexpr int RV = BMN / VEC;
#pragma unroll
  for (int i = 0; i < L::NVEC; ++i) {
    const int f = threadIdx.x + 256 * i;
    int off;
    int64_t k;
    if (KCONTIG) {
      off = kc_off<T>(f / 4, f % 4);
      k = k0 + (f % 4) * VEC;
    } else {
      off = mnc_off<T, BMN>(f / RV, f % RV);
      k = k0 + f / RV;
    }
    *reinterpret_cast<typename MF<T>::vec_t*>(tile + off) = k < kend ? r.v[i] : typename MF<T>::vec_t(0);
  }
}

// Block tile BM x BN (128 or 256 each; 128 x 128 for float64), 4 waves in a
// 2 x 2 grid of (BM/2) x (BN/2) wave tiles.
template <typename T, int BM, int BN, bool AKC, bool BKC>
__global__ void __launch_bounds__(256, (BM + BN > 384 ? 1 : 2)) gemm_dma_kernel(GemmArgs a) {
  using MFT = MF<T>;
  constexpr int BK = 64 / (int)sizeof(T);
  constexpr int MT = MFT::MT, VEC = MFT::VEC, LV = VEC == 4 ? 2 : 1;  // VEC = 1 << LV
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int TM = WM / MT, TN = WN / MT, NCH = BK / kKC;
  constexpr int TILE_A = BM * BK, TILE_B = BN * BK;  // elements per operand tile
  constexpr int NST = kDmaStages;
  __shared__ __attribute__((aligned(1024))) T lds[NST * (TILE_A + TILE_B)];

  int tm, tn;
  tile_coords(a, tm, tn);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int split = blockIdx.y;
  const int64_t batch = blockIdx.z;
  const int64_t kbeg = (int64_t)split * a.k_per_split;
  const int64_t kend = kbeg + a.k_per_split < a.K ? kbeg + a.k_per_split : a.K;
  const T* A = (const T*)a.A + batch * a.sA;
  const T* B = (const T*)a.B + batch * a.sB;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane / MT, c = lane % MT;
  const int wm0 = (wave >> 1) * WM, wn0 = (wave & 1) * WN;

  typename MFT::acc_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = typename MFT::acc_t(0);

  const int ntiles = kend > kbeg ? (int)((kend - kbeg + BK - 1) / BK) : 0;
  const int nfull = kend > kbeg ? (int)((kend - kbeg) / BK) : 0;
  DmaSrc<T, AKC, BM> sa;
  DmaSrc<T, BKC, BN> sb;
  dma_init<T, AKC, BM>(sa, A, a.lda, m0, a.M, kbeg, wave, lane);
  dma_init<T, BKC, BN>(sb, B, a.ldb, n0, a.N, kbeg, wave, lane);
  auto tileA = [&](int st) { return lds + st * (TILE_A + TILE_B); };
  auto tileB = [&](int st) { return lds + st * (TILE_A + TILE_B) + TILE_A; };
  // LDS byte address of this wave's first A chunk and first B chunk in stage
  // 0 (the low 32 bits of a generic LDS address are the LDS offset)
  const unsigned lds0 = (unsigned)(uintptr_t)lds;
  const unsigned ldsA = __builtin_amdgcn_readfirstlane(lds0 + wave * DmaSrc<T, AKC, BM>::NQ * 1024u);
  const unsigned ldsB =
      __builtin_amdgcn_readfirstlane(lds0 + TILE_A * (unsigned)sizeof(T) + wave * DmaSrc<T, BKC, BN>::NQ * 1024u);
  constexpr int STAGE_BYTES = (TILE_A + TILE_B) * (int)sizeof(T);
  constexpr int NQT = DmaSrc<T, AKC, BM>::NQ + DmaSrc<T, BKC, BN>::NQ;  // loads per wave per k-tile

  // Per-lane fragment offsets within a tile: KC fragment (rows base + c,
  // k-vector (8 / VEC) ch + g); MNC fragment element s (k-row
  // 8 ch + VEC g + s, column base + c).
  auto frag = [&](const T* __restrict__ t, bool kcontig, int bmn, int base, int ch) {
    typename MFT::vec_t v;
    if (kcontig) {
      v = *reinterpret_cast<const typename MFT::vec_t*>(t + kc_off<T>(base + c, (kKC / VEC) * ch + g));
    } else {
      const int n = base + c;
#pragma unroll
      for (int s = 0; s < VEC; ++s) {
        const int k = kKC * ch + VEC * g + s;
        v[s] = t[(bmn == 256 ? mnc_off<T, 256>(k, n >> LV) : mnc_off<T, 128>(k, n >> LV)) + (n & (VEC - 1))];
      }
    }
    return v;
  };
  const bool take_colsum = a.colsum != nullptr && tm == 0 && (int)threadIdx.x < BN;
  double csum = 0.0;
  auto compute = [&](int st) {
    const T* As = tileA(st);
    const T* Bs = tileB(st);  // st is a constant in the main loop: immediate LDS offsets
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
      typename MFT::vec_t fa[TM], fb[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) fa[i] = frag(As, AKC, BM, wm0 + i * MT, ch);
#pragma unroll
      for (int j = 0; j < TN; ++j) fb[j] = frag(Bs, BKC, BN, wn0 + j * MT, ch);
#pragma unroll
      for (int s = 0; s < VEC; ++s)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] = MFT::mma(fa[i][s], fb[j][s], acc[i][j]);
    }
    if (take_colsum) {
      // this thread's column of the B tile, its BK values in k order, then
      // into the running float64 sum (k past kend was stored as zero)
      const int n = threadIdx.x;
      T t = T(0);
#pragma unroll
      for (int k = 0; k < BK; ++k)
        t = t + (BKC ? Bs[kc_off<T>(n, k >> LV) + (k & (VEC - 1))] : Bs[mnc_off<T, BN>(k, n >> LV) + (n & (VEC - 1))]);
      csum += (double)t;
    }
  };

  static_assert(NST == 3, "the main loop is unrolled over three stages");
  auto issue = [&](auto stc) {
    constexpr int st = decltype(stc)::value;
    dma_issue<st * STAGE_BYTES>(sa, ldsA);
    dma_issue<st * STAGE_BYTES>(sb, ldsB);
  };
  // One k-tile: this wave's loads of tile kt have landed (the next tile's
  // may still be in flight), then every wave's have, and every wave is done
  // with the stage about to be refilled (that of tile kt - 1); then the
  // loads of tile kt + 2 and the MFMAs of tile kt.
  auto step = [&](auto stc, int kt) {
    constexpr int st = decltype(stc)::value;
    if (kt + 1 < nfull)
      dma_wait_barrier<NQT>();
    else
      dma_wait_barrier<0>();
    if (kt + 2 < nfull) issue(IC<(st + 2) % 3>());
    compute(st);
  };
  if (nfull > 0) issue(IC<0>());
  if (nfull > 1) issue(IC<1>());
  int kt = 0;
  for (; kt + 3 <= nfull; kt += 3) {
    step(IC<0>(), kt);
    step(IC<1>(), kt + 1);
    step(IC<2>(), kt + 2);
  }
  if (kt < nfull) step(IC<0>(), kt);
  if (kt + 1 < nfull) step(IC<1>(), kt + 1);
  const int st = nfull % 3;  // stage of the partial tile, if any
  if (ntiles > nfull) {  // the partial last k-tile, through registers
    const int64_t k0 = kbeg + (int64_t)nfull * BK;
    TilePtr<T, AKC, BM> pa;
    TilePtr<T, BKC, BN> pb;
    TileRegs<T, AKC, BM> ra;
    TileRegs<T, BKC, BN> rb;
    init_ptr<T, AKC, BM>(pa, A, a.lda, m0, a.M, k0);
    init_ptr<T, BKC, BN>(pb, B, a.ldb, n0, a.N, k0);
    load_tail<T, AKC, BM>(ra, pa, a.lda, k0, kend);
    load_tail<T, BKC, BN>(rb, pb, a.ldb, k0, kend);
    __syncthreads();  // every wave is done with the stage being refilled
    dma_tail_store<T, AKC, BM>(tileA(st), ra, k0, kend);
    dma_tail_store<T, BKC, BN>(tileB(st), rb, k0, kend);
    __syncthreads();
    compute(st);
  }
  if (take_colsum) finish_colsum<T>(a, csum, n0 + threadIdx.x, split);
  write_acc<T, TM, TN, true>(a, acc, m0 + wm0, n0 + wn0, g, c, split, batch);
}

// ---------------------------------------------------------------------------
// float32 products on the bf16 matrix cores (v_mfma_f32_32x32x16_bf16).
//
// A float32 x is the exact sum of three bf16 values: x0 = bf16(x), x1 =
// bf16(x - x0), x2 = x - x0 - x1 (round-to-nearest-even each time; x has 24
// significant bits and each step takes the leading 8, so x2 is left with at
// most 8 and bf16 holds it exactly). Then a*b = sum of the 9 products a_i b_j,
// each exact in float32 (8-bit by 8-bit significands). The kernel adds the 6
// with i + j <= 2 into float32 MFMA accumulators, smallest first, and drops
// a1 b2, a2 b1 and a2 b2: |a1| <= 2^-8 |a| and |a2| <= 2^-16 |a|, so what is
// dropped is below 2^-23 |a b| (about one float32 rounding of the product).
// The bf16 MFMA runs 16x the float32 MFMA's rate, so the 6 products take
// 3/8 of the matrix-core time of one float32 MFMA product.
//
// Data path: global float32 -> registers (16-byte vectors along k, or 8-byte
// vectors along m/n for m/n-contiguous operands, 4 k-rows at a time) ->
// split (v_cvt_pk_bf16_f32, two values per instruction) -> LDS as three bf16
// planes per operand, each [row][16 k] with the two 16-byte k-halves of a row
// swapped by a row swizzle, so the MFMA fragment reads (ds_read_b128: lane
// (g, c) reads row c, k 8g..8g+7) hit distinct banks.
// k-tile 16 (one MFMA k-step), two LDS stages, one barrier per k-tile.
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
constexpr int kX6BK = 16;

// x and y as three packed bf16 pairs (low half = x): p0 + p1 + p2 == (x, y) exactly.
// One v_cvt_pk_bf16_f32 per level; the two halves are widened back to float32
// by bit operations on the packed result (<< 16, & 0xffff0000).
// (as an asm statement: written as two __bf16 conversions, the compiler
// rebuilds the low half from a separate one-value conversion)
__device__ __forceinline__ unsigned cvt_pk_bf16(float x, float y) {
  unsigned r;
  asm("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(r) : "v"(x), "v"(y));
  return r;
}
__device__ __forceinline__ void split3(float x, float y, unsigned& p0, unsigned& p1, unsigned& p2) {
  p0 = cvt_pk_bf16(x, y);
  const float rx = x - __uint_as_float(p0 << 16), ry = y - __uint_as_float(p0 & 0xffff0000u);
  p1 = cvt_pk_bf16(rx, ry);
  p2 = cvt_pk_bf16(rx - __uint_as_float(p1 << 16), ry - __uint_as_float(p1 & 0xffff0000u));
}

// The two 16-byte k-halves of a plane row are swapped when bit 2 xor bit 3
// of the row is set: 8 consecutive rows (and 16) then cover distinct 16-byte
// bank groups, so 16-byte accesses by consecutive rows are conflict-free
// whether the LDS serves them 8 or 16 lanes at a time.
__device__ __forceinline__ int x6_swz(int row) { return ((row >> 2) ^ (row >> 3)) & 1; }
// byte offset of k-quad kq (k = 4kq..4kq+3) of `row` in one bf16 plane
__device__ __forceinline__ int x6_quad_off(int row, int kq) {
  return row * 32 + 16 * ((kq >> 1) ^ x6_swz(row)) + 8 * (kq & 1);
}
// byte offset of lane group g's 8 k-values (k = 8g..8g+7) of `row`
__device__ __forceinline__ int x6_frag_off(int row, int g) { return row * 32 + 16 * (g ^ x6_swz(row)); }

// Splits the 4 consecutive-k values v of `row` (k-quad kq) into the 3 planes.
template <int PLANE>
__device__ __forceinline__ void x6_store_quad(char* __restrict__ lds, int row, int kq, float v0, float v1, float v2,
                                              float v3) {
  unsigned a0, a1, a2, b0, b1, b2;
  split3(v0, v1, a0, a1, a2);
  split3(v2, v3, b0, b1, b2);
  typedef unsigned u2 __attribute__((ext_vector_type(2)));
  const int o = x6_quad_off(row, kq);
  *reinterpret_cast<u2*>(lds + o) = u2{a0, b0};
  *reinterpret_cast<u2*>(lds + PLANE + o) = u2{a1, b1};
  *reinterpret_cast<u2*>(lds + 2 * PLANE + o) = u2{a2, b2};
}

// Splits the 8 consecutive-k values x of `row` (k-half h: k = 8h..8h+7) into
// the 3 planes: one 16-byte store per plane.
template <int PLANE>
__device__ __forceinline__ void x6_store_oct(char* __restrict__ lds, int row, int h, const float (&x)[8]) {
  typedef unsigned u4 __attribute__((ext_vector_type(4)));
  u4 p0, p1, p2;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    unsigned a0, a1, a2;
    split3(x[2 * e], x[2 * e + 1], a0, a1, a2);
    p0[e] = a0;
    p1[e] = a1;
    p2[e] = a2;
  }
  const int o = x6_frag_off(row, h);
  *reinterpret_cast<u4*>(lds + o) = p0;
  *reinterpret_cast<u4*>(lds + PLANE + o) = p1;
  *reinterpret_cast<u4*>(lds + 2 * PLANE + o) = p2;
}

// One operand's BMN x 16 float32 tile. KCONTIG: NV = BMN/64 16-byte vectors
// per thread (row f/4, k-quad f%4). Otherwise NV = BMN/128 slots per thread of
// one column (f % BMN) x 8 k-rows (k-half f / BMN), 4-byte loads (a wave
// reads 64 consecutive columns of a k-row) and one 16-byte LDS store per
// plane (a wave writes 64 consecutive rows: conflict-free). Addresses are a
// wave-uniform base (advanced one k-tile per load, in scalar registers) plus
// per-thread 32-bit byte offsets fixed for the whole k loop; rows or columns
// past the matrix edge are clamped onto the last ones (they feed only
// outputs that are never stored). The host keeps every offset below 2^32
// (leading dimension < 2^22 elements).
template <bool KCONTIG, int BMN>
struct X6Src {
  static constexpr int NV = KCONTIG ? BMN / 64 : BMN / 128;
  static constexpr int NF = KCONTIG ? 1 : 8;  // loads per vector slot
  typedef typename std::conditional<KCONTIG, MF<float>::vec_t, float>::type ld_t;
  const char* base;
  unsigned off[NV];
  int64_t ldb;   // bytes between k-rows (n-contiguous operands)
  int64_t step;  // bytes per k-tile
  ld_t v[NV][NF];

  __device__ __forceinline__ void init(const float* __restrict__ P, int64_t ld, int64_t mn0, int64_t MN,
                                       int64_t kbeg) {
    base = reinterpret_cast<const char*>(KCONTIG ? P + mn0 * ld + kbeg : P + kbeg * ld + mn0);
    ldb = ld * 4;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int f = threadIdx.x + 256 * i;
      if constexpr (KCONTIG) {
        int64_t mn = mn0 + f / 4;
        mn = mn < MN ? mn : MN - 1;
        off[i] = (unsigned)(((mn - mn0) * ld + 4 * (f % 4)) * 4);
      } else {
        int64_t mn = mn0 + f % BMN;
        mn = mn < MN ? mn : MN - 1;
        off[i] = (unsigned)((8 * (f / BMN) * ld + (mn - mn0)) * 4);
      }
    }
    step = (KCONTIG ? (int64_t)kX6BK : (int64_t)kX6BK * ld) * 4;
  }
  // a k-tile wholly inside [kbeg, kend)
  __device__ __forceinline__ void load() {
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
      for (int j = 0; j < NF; ++j) v[i][j] = *reinterpret_cast<const ld_t*>(base + j * ldb + off[i]);
    base += step;
  }
  // the last k-tile, k0 + 16 > kend (k0 = its first k, kend - k0 a multiple
  // of 4): addresses clamped to the last k-quad (or k-row kend - 1), values
  // at k >= kend zeroed
  __device__ __forceinline__ void load_tail(int64_t k0, int64_t kend) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int f = threadIdx.x + 256 * i;
      if constexpr (KCONTIG) {
        const int64_t k = k0 + 4 * (f % 4);
        const int64_t back = k < kend ? 0 : (k - (kend - 4)) * 4;
        const ld_t x = *reinterpret_cast<const ld_t*>(base + off[i] - back);
        v[i][0] = k < kend ? x : ld_t(0);
      } else {
        const int h = f / BMN;
        const int64_t col_off = (int64_t)off[i] - 8 * h * ldb;  // the column's byte offset in a k-row
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int64_t k = k0 + 8 * h + j;
          const int64_t kr = (k < kend ? k : kend - 1) - k0;  // k-row within the tile, clamped
          const ld_t x = *reinterpret_cast<const ld_t*>(base + kr * ldb + col_off);
          v[i][j] = k < kend ? x : ld_t(0);
        }
      }
    }
  }
  // split the registers into the three planes of the LDS tile
  __device__ __forceinline__ void store(char* __restrict__ lds) const {
    constexpr int PLANE = BMN * 32;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int f = threadIdx.x + 256 * i;
      if constexpr (KCONTIG) {
        x6_store_quad<PLANE>(lds, f / 4, f % 4, v[i][0][0], v[i][0][1], v[i][0][2], v[i][0][3]);
      } else {
        float x[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = v[i][j];
        x6_store_oct<PLANE>(lds, f % BMN, f / BMN, x);
      }
    }
  }
  // column sums of an n-contiguous B tile: this thread's column over its 8
  // k-rows, in k order, into the running float64 sum
  __device__ __forceinline__ void colsum(double& cs) const {
    static_assert(!KCONTIG && NV == 1, "column sums: n-contiguous B, 128 columns");
    float t = v[0][0];
#pragma unroll
    for (int j = 1; j < 8; ++j) t = t + v[0][j];
    cs += (double)t;
  }
};

// Block tile BM x BN = 128 x 128, 4 waves in a 2 x 2 grid of 64 x 64 wave tiles.
template <int BM, int BN, bool AKC, bool BKC>
__global__ void __launch_bounds__(256, 3) gemm_x6_kernel(GemmArgs a) {
  static_assert(BM == 128 && BN == 128, "gemm_x6_kernel: 128 x 128 tiles");
  using MFT = MF<float>;
  constexpr int MT = 32, WM = BM / 2, WN = BN / 2, TM = WM / MT, TN = WN / MT;
  constexpr int A_BYTES = 3 * BM * 32, B_BYTES = 3 * BN * 32, STAGE = A_BYTES + B_BYTES;
  __shared__ __attribute__((aligned(16))) char lds[2 * STAGE];

  int tm, tn;
  tile_coords(a, tm, tn);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int split = blockIdx.y;
  const int64_t batch = blockIdx.z;
  const int64_t kbeg = (int64_t)split * a.k_per_split;
  const int64_t kend = kbeg + a.k_per_split < a.K ? kbeg + a.k_per_split : a.K;
  const float* A = (const float*)a.A + batch * a.sA;
  const float* B = (const float*)a.B + batch * a.sB;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane / MT, c = lane % MT;
  const int wm0 = (wave >> 1) * WM, wn0 = (wave & 1) * WN;

  MFT::acc_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = MFT::acc_t(0);

  const int64_t ntiles = kend > kbeg ? (kend - kbeg + kX6BK - 1) / kX6BK : 0;
  const int64_t nfull = kend > kbeg ? (kend - kbeg) / kX6BK : 0;
  X6Src<AKC, BM> sa;
  X6Src<BKC, BN> sb;
  sa.init(A, a.lda, m0, a.M, kbeg);
  sb.init(B, a.ldb, n0, a.N, kbeg);
  bool take_colsum = false;
  if constexpr (!BKC) take_colsum = a.colsum != nullptr && tm == 0;
  double cs = 0.0;
  auto store = [&](int stage) {
    sa.store(lds + stage * STAGE);
    sb.store(lds + stage * STAGE + A_BYTES);
    if constexpr (!BKC)
      if (take_colsum) sb.colsum(cs);
  };
  auto load_tail = [&](int64_t kt) {
    const int64_t k0 = kbeg + kt * kX6BK;
    sa.load_tail(k0, kend);
    sb.load_tail(k0, kend);
  };
  auto compute = [&](int stage) {
    const char* As = lds + stage * STAGE;
    const char* Bs = As + A_BYTES;
    bf16x8_t fa[TM][3], fb[TN][3];
#pragma unroll
    for (int p = 0; p < 3; ++p) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
        fa[i][p] = *reinterpret_cast<const bf16x8_t*>(As + p * (BM * 32) + x6_frag_off(wm0 + i * MT + c, g));
#pragma unroll
      for (int j = 0; j < TN; ++j)
        fb[j][p] = *reinterpret_cast<const bf16x8_t*>(Bs + p * (BN * 32) + x6_frag_off(wn0 + j * MT + c, g));
    }
    // partial products smallest first: (2,0) (1,1) (0,2) (1,0) (0,1) (0,0)
    constexpr int PA[6] = {2, 1, 0, 1, 0, 0}, PB[6] = {0, 1, 2, 0, 1, 0};
#pragma unroll
    for (int t = 0; t < 6; ++t)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i][PA[t]], fb[j][PB[t]], acc[i][j], 0, 0, 0);
  };
  if (ntiles > 0) {
    if (nfull > 0) {
      sa.load();
      sb.load();
    } else {
      load_tail(0);
    }
    store(0);
  }
  __syncthreads();
  // full k-tiles: the next tile is full too (no bounds work in this loop)
  int64_t kt = 0;
  for (; kt + 1 < nfull; ++kt) {
    sa.load();
    sb.load();
    compute((int)(kt & 1));
    store((int)(kt & 1) ^ 1);
    __syncthreads();
  }
  // the last full tile (its successor, if any, is the partial tail) and the tail
  for (; kt < ntiles; ++kt) {
    const bool more = kt + 1 < ntiles;
    if (more) load_tail(kt + 1);
    compute((int)(kt & 1));
    if (more) store((int)(kt & 1) ^ 1);
    __syncthreads();
  }
  if constexpr (!BKC) {
    if (take_colsum) {
      // the 2 threads of a column (k-halves 0, 1) add in k order
      double* red = reinterpret_cast<double*>(lds);
      red[threadIdx.x] = cs;
      __syncthreads();
      if ((int)threadIdx.x < BN) {
        const int n = threadIdx.x;
        finish_colsum<float>(a, red[n] + red[BN + n], n0 + n, split);
      }
    }
  }
  write_acc<float, TM, TN, true>(a, acc, m0 + wm0, n0 + wn0, g, c, split, batch);
}

// Sum of the split-K partials in split order 0, 1, ..., S-1, then the
// epilogue. PLAIN (bias only): VEC consecutive columns per thread.
template <typename T, bool PLAIN, int VEC>
__global__ void __launch_bounds__(256) splitk_reduce_kernel(GemmArgs a, const T* __restrict__ ws, int splits,
                                                             int64_t batch) {
  const int64_t M = a.M, N = a.N;
  const int64_t total = batch * M * N;
  const int64_t nvec = total / VEC;  // VEC divides N
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const T* __restrict__ bias = (const T*)a.bias;
  if (a.colsum_ws) {  // column sums of the splits, in split order
    T* cs = (T*)a.colsum;
    const T* w = (const T*)a.colsum_ws;
    for (int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; n < N; n += stride) {
      T v = w[n];
      for (int s = 1; s < splits; ++s) v = v + w[(int64_t)s * N + n];
      cs[n] = a.colsum_accumulate ? cs[n] + v : v;
    }
  }
  for (int64_t iv = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; iv < nvec; iv += stride) {
    const int64_t idx = iv * VEC;
    const int64_t b = idx / (M * N);
    const int64_t rem = idx - b * M * N;
    const int64_t m = rem / N, n = rem - m * N;
    T* C = (T*)a.C + b * a.sC;
    if (VEC > 1) {  // 16-byte vectors: every operand is aligned (checked by the host)
      typedef T vt __attribute__((ext_vector_type(VEC)));
      vt v = *reinterpret_cast<const vt*>(ws + idx);
      // four partials loaded at a time, added in split order
      int s = 1;
      for (; s + 3 < splits; s += 4) {
        vt t[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) t[u] = *reinterpret_cast<const vt*>(ws + (int64_t)(s + u) * total + idx);
#pragma unroll
        for (int u = 0; u < 4; ++u) v = v + t[u];
      }
      for (; s < splits; ++s) v = v + *reinterpret_cast<const vt*>(ws + (int64_t)s * total + idx);
      if (bias) v = v + *reinterpret_cast<const vt*>(bias + n);
      const int64_t o = m * a.ldc + n;
      if (!PLAIN) {  // the epilogue_store sequence, VEC elements at a time
        if (a.addend) v = *reinterpret_cast<const vt*>((const T*)a.addend + b * a.sC + o) + v;
        if (a.accumulate) v = *reinterpret_cast<const vt*>(C + o) + v;
        if (a.epi == kEpiGeluFwd) {
          vt y;
#pragma unroll
          for (int e = 0; e < VEC; ++e) y[e] = gelu_f<T>(v[e]);
          *reinterpret_cast<vt*>((T*)a.aux + b * a.sC + o) = y;
        } else if (a.epi == kEpiGeluBwd) {
          const vt x = *reinterpret_cast<const vt*>((const T*)a.aux + b * a.sC + o);
#pragma unroll
          for (int e = 0; e < VEC; ++e) v[e] = gelu_b<T>(x[e], v[e]);
        }
      }
      *reinterpret_cast<vt*>(C + o) = v;
      continue;
    }
    T v[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) v[e] = ws[idx + e];
    for (int s = 1; s < splits; ++s) {
      const T* w = ws + (int64_t)s * total + idx;
#pragma unroll
      for (int e = 0; e < VEC; ++e) v[e] = v[e] + w[e];
    }
    if (PLAIN) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) C[m * a.ldc + n + e] = bias ? v[e] + bias[n + e] : v[e];
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) epilogue_store<T>(a, C, a.ldc, m, n + e, v[e], b);
    }
  }
}

// Row dots of a float32 product whose rows are H = N / 64 groups of 64
// columns -- the attention output's gradient dO = dY W^T of the projection
// that reads the attention output X = O -- with X: rowdot[(b H + h) T + t] =
// sum_d C[m, 64 h + d] X[m, 64 h + d] for row m = b T + t, the rowsum(dO * O)
// term of the attention backward. Summed as the attention backward's own
// row pass sums it (four products in order, then a 16-lane butterfly), so the
// bits are that pass's. splitk_rowdot_kernel also forms C as the plain
// split-K sum (splitk_reduce_kernel's order); rowdot64_kernel reads a finished
// C. 16 consecutive threads cover one (row, group): N % 64 == 0.
__device__ __forceinline__ void rowdot_group(float d, int64_t idx, int64_t N, int64_t T, float* __restrict__ rowdot) {
#pragma unroll
  for (int off = 8; off >= 1; off >>= 1) d += __shfl_xor(d, off, 16);
  if ((threadIdx.x & 15) == 0) {
    const int64_t m = idx / N, h = (idx - m * N) / 64, b = m / T, t = m - b * T;
    rowdot[(b * (N / 64) + h) * T + t] = d;
  }
}

__global__ void __launch_bounds__(256) splitk_rowdot_kernel(GemmArgs a, const float* __restrict__ ws, int splits,
                                                             const float* __restrict__ X, float* __restrict__ rowdot,
                                                             int64_t T) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  const int64_t N = a.N, total = a.M * N, nvec = total / 4;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  float* C = (float*)a.C;
  for (int64_t iv = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; iv < nvec; iv += stride) {
    const int64_t idx = iv * 4;
    // X and the first two partials in flight together
    const f4 o = *reinterpret_cast<const f4*>(X + idx);
    f4 v = *reinterpret_cast<const f4*>(ws + idx);
    const f4 p1 = *reinterpret_cast<const f4*>(ws + total + idx);  // splits >= 2
    v = v + p1;
    int s = 2;
    for (; s + 3 < splits; s += 4) {
      f4 t[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) t[u] = *reinterpret_cast<const f4*>(ws + (int64_t)(s + u) * total + idx);
#pragma unroll
      for (int u = 0; u < 4; ++u) v = v + t[u];
    }
    for (; s < splits; ++s) v = v + *reinterpret_cast<const f4*>(ws + (int64_t)s * total + idx);
    *reinterpret_cast<f4*>(C + idx) = v;
    rowdot_group(((o[0] * v[0] + o[1] * v[1]) + o[2] * v[2]) + o[3] * v[3], idx, N, T, rowdot);
  }
}

__global__ void __launch_bounds__(256) rowdot64_kernel(const float* __restrict__ C, const float* __restrict__ X,
                                                        float* __restrict__ rowdot, int64_t M, int64_t N, int64_t T) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  const int64_t nvec = M * N / 4;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t iv = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; iv < nvec; iv += stride) {
    const int64_t idx = iv * 4;
    const f4 v = *reinterpret_cast<const f4*>(C + idx);
    const f4 o = *reinterpret_cast<const f4*>(X + idx);
    rowdot_group(((o[0] * v[0] + o[1] * v[1]) + o[2] * v[2]) + o[3] * v[3], idx, N, T, rowdot);
  }
}

// Split-K sum, bias and residual of an output row, then the LayerNorm of the
// finished row, in one pass: one wave per row, the row in registers. The
// output element is (((p_0 + p_1) + ...) + bias) then residual + that -- the
// reduction kernel's and epilogue's order -- and the LayerNorm is the shared
// row code of the LayerNorm kernel, so C, ln_out, mean and rstd are the bits
// the separate kernels give. 16-byte aligned rows, unbatched. S2: exactly
// two partials (the common split), loaded with no stand-in re-reads.
template <typename T, int NV, int VW, bool S2>
__global__ void __launch_bounds__(256) splitk_ln_kernel(GemmArgs a, const T* __restrict__ ws, int splits,
                                                         T* __restrict__ hout, T* __restrict__ mean,
                                                         T* __restrict__ rstd, const T* __restrict__ lw,
                                                         const T* __restrict__ lb, T eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t M = a.M;
  const int cols = (int)a.N;
  if (row >= M) return;
  const int64_t total = M * a.N;
  const T* bias = (const T*)a.bias;
  const T* add = (const T*)a.addend;
  T* C = (T*)a.C;
  // every load of the row is issued before the first add, from addresses
  // that are always valid (a missing split, bias or residual re-reads the
  // first partial and is then left out), so no load waits behind a branch
  constexpr int SP = S2 ? 2 : (NV * VW <= 16 ? 4 : (NV * VW <= 32 ? 2 : 1));
  if (S2) splits = 2;
  T pv[SP][NV][VW], bv[NV][VW], rv[NV][VW];
  const T* bsrc = bias ? bias : ws;
  const T* rsrc = add ? add + row * a.ldc : ws + row * a.N;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = VW * lane + 64 * VW * j;
    const int cc = c < cols ? c : 0;
    const int64_t idx = row * a.N + cc;
#pragma unroll
    for (int sp = 0; sp < SP; ++sp) load_vec<T, VW>(pv[sp][j], ws + (int64_t)(sp < splits ? sp : 0) * total + idx);
    load_vec<T, VW>(bv[j], bsrc + cc);
    load_vec<T, VW>(rv[j], rsrc + cc);
  }
  T xv[NV][VW];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = VW * lane + 64 * VW * j;
    T v[VW];
#pragma unroll
    for (int e = 0; e < VW; ++e) v[e] = pv[0][j][e];
#pragma unroll
    for (int sp = 1; sp < SP; ++sp)
      if (sp < splits)
#pragma unroll
        for (int e = 0; e < VW; ++e) v[e] = v[e] + pv[sp][j][e];
    if (c < cols) {
      for (int sp = SP; sp < splits; ++sp) {  // more splits than held in registers
        T t[VW];
        load_vec<T, VW>(t, ws + (int64_t)sp * total + row * a.N + c);
#pragma unroll
        for (int e = 0; e < VW; ++e) v[e] = v[e] + t[e];
      }
    }
    if (bias)
#pragma unroll
      for (int e = 0; e < VW; ++e) v[e] = v[e] + bv[j][e];
    if (add)
#pragma unroll
      for (int e = 0; e < VW; ++e) v[e] = rv[j][e] + v[e];
    if (c < cols) {
      store_vec<T, VW>(C + row * a.ldc + c, v);
#pragma unroll
      for (int e = 0; e < VW; ++e) xv[j][e] = v[e];
    } else {
#pragma unroll
      for (int e = 0; e < VW; ++e) xv[j][e] = T(0);
    }
  }
  ln_row_fwd<T, NV, VW>(xv, cols, lane, lw, lb, eps, hout + row * cols, mean + row, rstd + row);
}

template <typename T, int BM, int BN, bool AKC, bool BKC>
static void launch_variant(const GemmArgs& a, dim3 grid, bool veca, bool vecb, bool dma) {
  if (dma) {
    if constexpr (std::is_same<T, float>::value || (BM == 128 && BN == 128))
      gemm_dma_kernel<T, BM, BN, AKC, BKC><<<grid, 256, 0, stream()>>>(a);
    return;
  }
  if constexpr (BM != 128 || BN != 128) return;  // larger tiles: aligned float32 only (see gemm_impl)
  if (veca && vecb)
    gemm_kernel<T, BM, BN, AKC, BKC, true, true><<<grid, 256, 0, stream()>>>(a);
  else if (veca)
    gemm_kernel<T, BM, BN, AKC, BKC, true, false><<<grid, 256, 0, stream()>>>(a);
  else if (vecb)
    gemm_kernel<T, BM, BN, AKC, BKC, false, true><<<grid, 256, 0, stream()>>>(a);
  else
    gemm_kernel<T, BM, BN, AKC, BKC, false, false><<<grid, 256, 0, stream()>>>(a);
}

static void launch_x6(const GemmArgs& a, dim3 grid, int akc, int bkc) {
  if (akc && bkc)
    gemm_x6_kernel<128, 128, true, true><<<grid, 256, 0, stream()>>>(a);
  else if (akc)
    gemm_x6_kernel<128, 128, true, false><<<grid, 256, 0, stream()>>>(a);
  else if (bkc)
    gemm_x6_kernel<128, 128, false, true><<<grid, 256, 0, stream()>>>(a);
  else
    gemm_x6_kernel<128, 128, false, false><<<grid, 256, 0, stream()>>>(a);
}

// float32 GEMM arithmetic: DTMI_GEMM_MATH_F32 (float32 MFMA) or
// DTMI_GEMM_MATH_BF16X6 (exact 3-way bf16 split, 6 bf16 MFMA products).
static int g_gemm_math = DTMI_GEMM_MATH_F32;

template <typename T, int BM, int BN>
static void launch_layout(const GemmArgs& a, dim3 grid, int akc, int bkc, bool veca, bool vecb, bool dma) {
  if (akc && bkc)
    launch_variant<T, BM, BN, true, true>(a, grid, veca, vecb, dma);
  else if (akc)
    launch_variant<T, BM, BN, true, false>(a, grid, veca, vecb, dma);
  else if (bkc)
    launch_variant<T, BM, BN, false, true>(a, grid, veca, vecb, dma);
  else
    launch_variant<T, BM, BN, false, false>(a, grid, veca, vecb, dma);
}

struct EpiArgs {
  const void* addend = nullptr;
  int epi = kEpiNone;
  void* aux = nullptr;
  void* colsum = nullptr;  // column sums of B (length N), unbatched
  int colsum_accumulate = 0;
  // Split-K partials left for the consumer: when the chooser takes between 2
  // and parts_max splits, the raw partials go to parts_out ([splits][M][N],
  // unbatched, no bias or epilogue) with no sum pass and *parts_n = splits;
  // otherwise C is written as usual and *parts_n = 1.
  void* parts_out = nullptr;
  int parts_max = 0;
  int* parts_n = nullptr;
  // float32 row dots with X per 64-column group (see splitk_rowdot_kernel)
  const void* rowdot_x = nullptr;
  void* rowdot_out = nullptr;
  int64_t rowdot_T = 1;
  // LayerNorm of the finished output rows (after bias and residual):
  // ln_out = layer_norm(C; ln_w, ln_b, ln_eps), with the row mean and rstd
  void* ln_out = nullptr;
  void* ln_mean = nullptr;
  void* ln_rstd = nullptr;
  const void* ln_w = nullptr;
  const void* ln_b = nullptr;
  double ln_eps = 1e-5;
};

// K splits. A grid of b blocks on C CUs runs ceil(b / C) rounds, so its
// useful fraction is b / (C * ceil(b / C)); take the fewest splits (each
// keeping >= 256 of K) that reach 90 % of rounds, else the best found. A grid
// of fewer than ~2 blocks per CU leaves one wave per SIMD, which cannot hide
// its own latencies: it counts 15 % less (measured: the 768 x 768 x 8192
// weight gradient ran at 114 TFLOP/s on 252 blocks).
static int choose_splits(int64_t tiles, int64_t batch, int64_t K, int64_t cus) {
  int splits = 1;
  double e_best = 0.0;
  for (int sp = 1; sp <= 16; ++sp) {
    if (sp > 1 && K / sp < 256) break;
    const int64_t blocks = tiles * batch * sp;
    double eff = (double)blocks / (double)(cus * cdiv(blocks, cus));
    if (10 * blocks < 19 * cus) eff *= 0.85;
    if (eff > e_best + 1e-9) {
      e_best = eff;
      splits = sp;
    }
    if (eff >= 0.9) break;
  }
  return splits;
}

// Block tile of the aligned float32 kernel: 256 x 128 when every block still
// gets a long k range (>= 1024) and the grid covers the CUs, else 128 x 128.
// The larger tile moves 25 % fewer bytes per MFMA through the loads and LDS
// but has half the blocks; on the GPT-2 shapes it wins for the long-K
// products (dW, the vocabulary head's dX and dW) and loses on K = 768. When
// the larger tile needs a K split and the smaller one fills whole rounds
// without one, the smaller one is taken: no partials, no sum pass.
static void pick_tile(int64_t M, int64_t N, int64_t K, int64_t batch, int64_t cus, int& bm, int& bn) {
  bm = bn = 128;
  if (M < 256) return;
  const int64_t tiles = cdiv(M, 256) * cdiv(N, 128);
  const int sp = choose_splits(tiles, batch, K, cus);
  if (tiles * batch * sp >= cus && K / sp >= 1024) bm = 256;
  if (bm == 256 && sp > 1) {
    const int64_t t128 = cdiv(M, 128) * cdiv(N, 128);
    if (choose_splits(t128, batch, K, cus) == 1 && t128 * batch % cus == 0) bm = 128;
  }
}

template <typename T>
static int gemm_impl(int akc, int bkc, int64_t M, int64_t N, int64_t K, const void* A, int64_t lda, int64_t sA,
                     const void* B, int64_t ldb, int64_t sB, void* C, int64_t ldc, int64_t sC, int64_t batch,
                     const void* bias, int accumulate, int force_splits, const EpiArgs& ep) {
  constexpr int VEC = MF<T>::VEC;
  GemmArgs a{};
  a.A = A;
  a.B = B;
  a.C = C;
  a.bias = bias;
  a.M = M;
  a.N = N;
  a.K = K;
  a.lda = lda;
  a.ldb = ldb;
  a.ldc = ldc;
  a.sA = sA;
  a.sB = sB;
  a.sC = sC;
  a.accumulate = accumulate;
  a.addend = ep.addend;
  a.epi = ep.epi;
  a.aux = ep.aux;
  a.colsum = ep.colsum;
  a.colsum_accumulate = ep.colsum_accumulate;
  const int64_t cus = num_cus() > 0 ? num_cus() : 256;
  const bool veca = aligned(A, 16) && lda % VEC == 0 && (batch == 1 || sA % VEC == 0) && (akc ? K % VEC == 0 : M % VEC == 0);
  const bool vecb = aligned(B, 16) && ldb % VEC == 0 && (batch == 1 || sB % VEC == 0) && (bkc ? K % VEC == 0 : N % VEC == 0);
  // The direct-to-LDS kernel addresses a tile with 32-bit byte offsets from
  // its origin: leading dimensions below 2^24 bytes keep them in range.
  constexpr int64_t kDmaMaxLd = (1 << 24) / (int64_t)sizeof(T);
  const bool dma = veca && vecb && lda < kDmaMaxLd && ldb < kDmaMaxLd;
  // split-bf16 products: aligned float32 operands (its column sums need an
  // n-contiguous B)
  const bool x6 = std::is_same<T, float>::value && veca && vecb && g_gemm_math == DTMI_GEMM_MATH_BF16X6 &&
                  !(a.colsum && bkc) && lda < (1 << 22) && ldb < (1 << 22);
  int bm = 128, bn = 128;
  if (std::is_same<T, float>::value && dma && !x6) pick_tile(M, N, K, batch, cus, bm, bn);
  const int64_t tmn = cdiv(M, bm) * cdiv(N, bn);
  int splits = force_splits > 0 ? force_splits : choose_splits(tmn, batch, K, cus);
  a.tiles_m = (int)cdiv(M, bm);
  a.tiles_n = (int)cdiv(N, bn);
  const int64_t tiles = (int64_t)a.tiles_m * a.tiles_n;
  DTMI_CHECK(tiles < (1LL << 31) && batch < 65536, "dtmi_gemm: problem too large");
  constexpr int kBK = kBKT<T>;
  int64_t kps = cdiv(cdiv(K, splits), kBK) * kBK;
  if (kps < kBK) kps = kBK;
  splits = (int)cdiv(K > 0 ? K : 1, kps);
  a.k_per_split = kps;
  const size_t es = sizeof(T);
  void* ws = nullptr;
  // the partials handed to the consumer (see EpiArgs::parts_out)
  const bool to_parts = ep.parts_out && splits > 1 && splits <= ep.parts_max && batch == 1 && !bias &&
                        !a.accumulate && a.epi == kEpiNone && !a.addend && !a.colsum && ldc == N;
  if (ep.parts_n) *ep.parts_n = to_parts ? splits : 1;
  if (to_parts) {
    a.ws = ep.parts_out;
  } else if (splits > 1) {
    const size_t main_bytes = (size_t)splits * batch * M * N * es;
    const size_t cs_bytes = a.colsum ? (size_t)splits * N * es : 0;
    int rc = pool_alloc(&ws, main_bytes + cs_bytes);
    if (rc) return rc;
    a.ws = ws;
    if (a.colsum) a.colsum_ws = (char*)ws + main_bytes;
  }
  // A LayerNorm of the output rows is fused into the split-K sum when the
  // rows fit the row kernel; otherwise it runs as its own pass afterwards.
  constexpr int LVW = 16 / sizeof(T);
  const int ln_nv = ep.ln_out ? ln_pick_nv(cdiv(N, 64LL * LVW)) : -1;
  const bool ln_fused = splits > 1 && ep.ln_out && batch == 1 && !a.accumulate && a.epi == kEpiNone &&
                        N % LVW == 0 && ldc == N && ln_nv > 0 && aligned(C, 16) && (!bias || aligned(bias, 16)) &&
                        (!a.addend || aligned(a.addend, 16)) && aligned(ep.ln_out, 16) && aligned(ep.ln_w, 16) &&
                        aligned(ep.ln_b, 16);
  // row dots of C with X fused into the split-K sum when C is a plain sum,
  // else a pass over the finished C
  const bool rowdot_fused = ep.rowdot_out && splits > 1 && batch == 1 && !bias && !a.addend && !a.accumulate &&
                            a.epi == kEpiNone && ldc == N && N % 64 == 0 && aligned(C, 16) &&
                            aligned(ep.rowdot_x, 16);
  bool rowdot_done = false;
  dim3 grid((unsigned)tiles, (unsigned)splits, (unsigned)batch);
  {
    TimedLaunch tl(DTMI_FAM_GEMM, 2.0 * (double)M * N * K * batch);
    if constexpr (std::is_same<T, float>::value) {
      if (x6)
        launch_x6(a, grid, akc, bkc);
      else if (bm == 256)
        launch_layout<T, 256, 128>(a, grid, akc, bkc, veca, vecb, dma);
      else if (bn == 256)
        launch_layout<T, 128, 256>(a, grid, akc, bkc, veca, vecb, dma);
      else
        launch_layout<T, 128, 128>(a, grid, akc, bkc, veca, vecb, dma);
    } else {
      launch_layout<T, 128, 128>(a, grid, akc, bkc, veca, vecb, dma);
    }
    if (splits > 1 && !ln_fused && !to_parts) {
      int64_t total = batch * M * N;
      int rg = (int)(cdiv(total, 256 * 4) < 8192 ? cdiv(total, 256 * 4) : 8192);
      GemmArgs r = a;
      r.ws = nullptr;
      const bool plain = a.addend == nullptr && a.epi == kEpiNone && !a.accumulate;
      constexpr int V = 16 / sizeof(T);
      const bool vec_ok = N % V == 0 && ldc % V == 0 && (batch == 1 || sC % V == 0) && aligned(C, 16) &&
                          (!bias || aligned(bias, 16)) && (!a.addend || aligned(a.addend, 16)) &&
                          (!a.aux || aligned(a.aux, 16));
      if constexpr (std::is_same<T, float>::value) {
        if (rowdot_fused) {
          splitk_rowdot_kernel<<<rg, 256, 0, stream()>>>(r, (const float*)ws, splits, (const float*)ep.rowdot_x,
                                                          (float*)ep.rowdot_out, ep.rowdot_T);
          rowdot_done = true;
        }
      }
      if (rowdot_done) {
      } else if (plain && vec_ok)
        splitk_reduce_kernel<T, true, V><<<rg, 256, 0, stream()>>>(r, (const T*)ws, splits, batch);
      else if (vec_ok)
        splitk_reduce_kernel<T, false, V><<<rg, 256, 0, stream()>>>(r, (const T*)ws, splits, batch);
      else if (plain)
        splitk_reduce_kernel<T, true, 1><<<rg, 256, 0, stream()>>>(r, (const T*)ws, splits, batch);
      else
        splitk_reduce_kernel<T, false, 1><<<rg, 256, 0, stream()>>>(r, (const T*)ws, splits, batch);
    }
  }
  if (ln_fused) {
    // split-K partials, bias and residual in; C and the LayerNorm out
    TimedLaunch tl(DTMI_FAM_OTHER, (double)M * N * sizeof(T) * (splits + (a.addend ? 3 : 2)));
    GemmArgs r = a;
    r.ws = nullptr;
    const unsigned lg = (unsigned)cdiv(M, 4);
#define CALL_LN_S(NV, S2)                                                                                      \
  splitk_ln_kernel<T, NV, LVW, S2><<<lg, 256, 0, stream()>>>(r, (const T*)ws, splits, (T*)ep.ln_out,               \
                                                              (T*)ep.ln_mean, (T*)ep.ln_rstd, (const T*)ep.ln_w, \
                                                              (const T*)ep.ln_b, (T)ep.ln_eps)
#define CALL_LN(NV)          \
  if (splits == 2)           \
    CALL_LN_S(NV, true);     \
  else                       \
    CALL_LN_S(NV, false)
    LN_NV_SWITCH(ln_nv, CALL_LN)
#undef CALL_LN
#undef CALL_LN_S
  }
  if constexpr (std::is_same<T, float>::value) {
    if (ep.rowdot_out && !rowdot_done) {
      TimedLaunch tl(DTMI_FAM_OTHER, 2.0 * (double)M * N * sizeof(T));
      const int64_t nv = M * N / 4;
      rowdot64_kernel<<<(unsigned)(cdiv(nv, 256) < 8192 ? cdiv(nv, 256) : 8192), 256, 0, stream()>>>(
          (const float*)C, (const float*)ep.rowdot_x, (float*)ep.rowdot_out, M, N, ep.rowdot_T);
    }
  }
  hipError_t le = hipGetLastError();
  if (ws) pool_free(ws);
  if (le != hipSuccess) return fail_hip(le, "gemm kernels", __FILE__, __LINE__);
  if (ep.ln_out && !ln_fused)  // the LayerNorm as its own pass over C
    return dtmi_layernorm_fwd(std::is_same<T, float>::value ? DTMI_F32 : DTMI_F64, ep.ln_out, ep.ln_mean, ep.ln_rstd,
                              C, ep.ln_w, ep.ln_b, M, N, ep.ln_eps);
  return DTMI_OK;
}

static int gemm_dispatch(int dtype, int akc, int bkc, int64_t M, int64_t N, int64_t K, const void* A, int64_t lda,
                         int64_t sA, const void* B, int64_t ldb, int64_t sB, void* C, int64_t ldc, int64_t sC,
                         int64_t batch, const void* bias, int accumulate, int force_splits,
                         const EpiArgs& ep = EpiArgs()) {
  DTMI_DTYPE_OK(dtype);
  DTMI_CHECK(M >= 0 && N >= 0 && K >= 0 && batch >= 1, "dtmi_gemm: bad sizes M=%lld N=%lld K=%lld batch=%lld",
             (long long)M, (long long)N, (long long)K, (long long)batch);
  if (M == 0 || N == 0) return DTMI_OK;
  DTMI_CHECK(C != nullptr && (K == 0 || (A && B)), "dtmi_gemm: NULL pointer");
  DTMI_CHECK(ldc >= N, "dtmi_gemm: ldc %lld < N %lld", (long long)ldc, (long long)N);
  DTMI_CHECK(K == 0 || (akc ? lda >= K : lda >= M), "dtmi_gemm: lda too small");
  DTMI_CHECK(K == 0 || (bkc ? ldb >= K : ldb >= N), "dtmi_gemm: ldb too small");
  DTMI_CHECK(ep.epi == kEpiNone || ep.aux != nullptr, "dtmi_gemm: GELU epilogue without its array");
  DTMI_CHECK(ep.colsum == nullptr || batch == 1, "dtmi_gemm: column sums are for unbatched products");
  if (dtype == DTMI_F32)
    return gemm_impl<float>(akc, bkc, M, N, K, A, lda, sA, B, ldb, sB, C, ldc, sC, batch, bias, accumulate,
                            force_splits, ep);
  return gemm_impl<double>(akc, bkc, M, N, K, A, lda, sA, B, ldb, sB, C, ldc, sC, batch, bias, accumulate,
                           force_splits, ep);
}

}  // namespace dtmi

using namespace dtmi;

DTMI_EXPORT int dtmi_set_gemm_math(int math) {
  DTMI_BODY_BEGIN
  DTMI_CHECK(math == DTMI_GEMM_MATH_F32 || math == DTMI_GEMM_MATH_BF16X6, "dtmi_set_gemm_math: unknown mode %d",
             math);
  g_gemm_math = math;
  return DTMI_OK;
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_get_gemm_math(int* math) {
  DTMI_BODY_BEGIN
  DTMI_CHECK(math != nullptr, "dtmi_get_gemm_math: NULL pointer");
  *math = g_gemm_math;
  return DTMI_OK;
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_gemm(int dtype, int a_kcontig, int b_kcontig, int64_t M, int64_t N, int64_t K, const void* A,
                          int64_t lda, int64_t strideA, const void* B, int64_t ldb, int64_t strideB, void* C,
                          int64_t ldc, int64_t strideC, int64_t batch, const void* bias, int accumulate,
                          int splits) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  return gemm_dispatch(dtype, a_kcontig ? 1 : 0, b_kcontig ? 1 : 0, M, N, K, A, lda, strideA, B, ldb, strideB, C, ldc,
                       strideC, batch, bias, accumulate, splits);
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_linear_fwd(int dtype, void* Y, const void* X, const void* W, const void* b, int64_t M,
                                int64_t K, int64_t N) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  return gemm_dispatch(dtype, 1, 0, M, N, K, X, K, 0, W, N, 0, Y, N, 0, 1, b, 0, 0);
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_linear_fwd_fused(int dtype, void* Y, void* act, const void* X, const void* W, const void* b,
                                      const void* residual, int64_t M, int64_t K, int64_t N) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  EpiArgs ep;
  ep.addend = residual;
  ep.epi = act ? kEpiGeluFwd : kEpiNone;
  ep.aux = act;
  DTMI_CHECK(!(act && residual), "dtmi_linear_fwd_fused: GELU and residual are not fused together");
  return gemm_dispatch(dtype, 1, 0, M, N, K, X, K, 0, W, N, 0, Y, N, 0, 1, b, 0, 0, ep);
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_linear_fwd_ln(int dtype, void* Y, void* H, void* mean, void* rstd, const void* X, const void* W,
                                   const void* b, const void* residual, const void* ln_w, const void* ln_b, double eps,
                                   int64_t M, int64_t K, int64_t N) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_CHECK(H && mean && rstd && ln_w && ln_b, "dtmi_linear_fwd_ln: NULL LayerNorm pointer");
  DTMI_CHECK(H != Y, "dtmi_linear_fwd_ln: the LayerNorm output must not be Y");
  EpiArgs ep;
  ep.addend = residual;
  ep.ln_out = H;
  ep.ln_mean = mean;
  ep.ln_rstd = rstd;
  ep.ln_w = ln_w;
  ep.ln_b = ln_b;
  ep.ln_eps = eps;
  return gemm_dispatch(dtype, 1, 0, M, N, K, X, K, 0, W, N, 0, Y, N, 0, 1, b, 0, 0, ep);
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_linear_bwd_dx_gelu(int dtype, void* dX, const void* dY, const void* W, const void* pre,
                                        int64_t M, int64_t K, int64_t N) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_CHECK(pre != nullptr, "dtmi_linear_bwd_dx_gelu: NULL pre-activation");
  EpiArgs ep;
  ep.epi = kEpiGeluBwd;
  ep.aux = const_cast<void*>(pre);
  return gemm_dispatch(dtype, 1, 1, M, K, N, dY, N, 0, W, N, 0, dX, K, 0, 1, nullptr, 0, 0, ep);
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_linear_bwd_dx(int dtype, void* dX, const void* dY, const void* W, int64_t M, int64_t K,
                                   int64_t N, int accumulate) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  // dX[m, k] = sum_n dY[m, n] W[k, n]: A = dY (k-contiguous over n), B(n, k) = W[k, n] (k-contiguous)
  return gemm_dispatch(dtype, 1, 1, M, K, N, dY, N, 0, W, N, 0, dX, K, 0, 1, nullptr, accumulate, 0);
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_linear_bwd_dx_parts(int dtype, void* parts, int max_parts, int* nparts, const void* dY,
                                         const void* W, int64_t M, int64_t K, int64_t N) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_CHECK(parts && nparts && max_parts >= 1, "dtmi_linear_bwd_dx_parts: NULL parts / nparts or max_parts < 1");
  EpiArgs ep;
  ep.parts_out = parts;
  ep.parts_max = max_parts;
  ep.parts_n = nparts;
  *nparts = 1;
  return gemm_dispatch(dtype, 1, 1, M, K, N, dY, N, 0, W, N, 0, parts, K, 0, 1, nullptr, 0, 0, ep);
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_linear_bwd_dx_rowdot(int dtype, void* dX, const void* dY, const void* W, const void* X,
                                          void* rowdot, int64_t M, int64_t K, int64_t N, int64_t T) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_CHECK(dtype == DTMI_F32, "dtmi_linear_bwd_dx_rowdot: float32 only");
  DTMI_CHECK(M >= 0 && K > 0 && N >= 0 && T > 0 && K % 64 == 0 && M % T == 0,
             "dtmi_linear_bwd_dx_rowdot: needs K %% 64 == 0 and M %% T == 0 (M=%lld K=%lld T=%lld)", (long long)M,
             (long long)K, (long long)T);
  DTMI_CHECK(X && rowdot && aligned(dX, 16) && aligned(X, 16), "dtmi_linear_bwd_dx_rowdot: NULL or unaligned X / dX");
  EpiArgs ep;
  ep.rowdot_x = X;
  ep.rowdot_out = rowdot;
  ep.rowdot_T = T;
  return gemm_dispatch(dtype, 1, 1, M, K, N, dY, N, 0, W, N, 0, dX, K, 0, 1, nullptr, 0, 0, ep);
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_linear_bwd_dw(int dtype, void* dW, void* db, const void* X, const void* dY, int64_t M,
                                   int64_t K, int64_t N, int accumulate) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  // dW[k, n] = sum_m X[m, k] dY[m, n]: A(k, m) = X[m, k] (k-major storage), B(m, n) = dY[m, n];
  // db[n] = sum_m dY[m, n], the column sums of B, taken inside the same GEMM
  if (K == 0) return db ? dtmi_colsum(dtype, db, dY, M, N, accumulate) : DTMI_OK;  // no dW tiles to carry db
  EpiArgs ep;
  ep.colsum = db;
  ep.colsum_accumulate = accumulate;
  return gemm_dispatch(dtype, 0, 0, K, N, M, X, K, 0, dY, N, 0, dW, N, 0, 1, nullptr, accumulate, 0, ep);
  DTMI_BODY_END
}
