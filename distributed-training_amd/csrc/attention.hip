// Causal self-attention on the MFMA cores: flash-style forward that keeps the
// per-row max and sum of the softmax, and a backward that recomputes the
// probabilities from them (dtrain/autograd.py:226-247 computes and keeps the
// full (B, H, T, T) probability tensor instead).
//
// Shapes (B, H, T, D) with D contiguous and arbitrary element strides for the
// b, h and t axes, so q/k/v are read straight out of the fused qkv projection
// ([B, T, 3, H, D] row-major) and o / dq / dk / dv are written straight into
// [B, T, H, D] / [B, T, 3, H, D] layouts: the reshape/transpose/split of
// dtrain/nn.py:100-103 costs no copies.
//
// Transposed formulation. With MT x MT MFMA tiles (32 in float32, 16 in
// float64) an MFMA result gives each lane one column and NACC rows. Each wave
// owns MT queries (forward, dQ) or MT keys (dK/dV) as the COLUMNS of its tiles
// (S^T = K Q^T in the forward), so per-query softmax statistics are per-lane
// values combined across the G lane groups with one or two xor-shuffles, and
// the probabilities computed in registers feed the next MFMA directly as its
// B operand: result register i of lane group g is exactly the value that lane
// supplies as k-slot g of an MFMA step, with the A operand (V, dO, K or Q
// rows) read from LDS at the matching row. The k-permutation is the same on
// both operands, so every product is a plain sum over the reduction index.
//
// Backward without atomics: kernel A owns keys and loops over the query tiles
// that see them, recomputing P = exp(s - max) / sum (dK, dV accumulate in
// registers) and writing dS = P * (dP - rowsum(dO * O)) to a [B, H, T, T]
// workspace; kernel B owns queries and accumulates dQ = dS K from it (when
// the workspace would exceed its bound, kernel B recomputes dS instead).
// Float32 with D = 64 and T a multiple of 32 works on 16 x 16 tiles with
// paired ranges: key tile j and its mirror nt - 1 - j (nt + 1 tile pairs
// between them) split over two waves in the key pass, query tile i and its
// mirror over a pair of waves in the dQ pass, so every wave carries the same
// work whatever the sequence length, and dS lives in causal tiles only.
// Otherwise a block owns 128 keys (queries), one 32-wide (16-wide in
// float64) tile per wave, and the float32 kernel A keeps its query and dO
// tiles also transposed in LDS so the dK / dV MFMAs read them with 16-byte
// vectors. Results are deterministic.
#include <cmath>

#include "bufrsrc.h"
#include "common.h"

namespace dtmi {

// One float64 through a buffer resource.
__device__ __forceinline__ double buf_load_f64(Rsrc r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(double, __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, (int)soff, 0));
}

template <typename T>
struct AM;
template <>
struct AM<float> {
  static constexpr int MT = 32, G = 2, VEC = 4, NACC = 16, PAD = 4;
  typedef float acc_t __attribute__((ext_vector_type(16)));
  typedef float vec_t __attribute__((ext_vector_type(4)));
  static __device__ __forceinline__ acc_t mma(float a, float b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ int row(int i, int g) { return 8 * (i / 4) + 4 * g + (i % 4); }
};
template <>
struct AM<double> {
  static constexpr int MT = 16, G = 4, VEC = 2, NACC = 4, PAD = 2;
  typedef double acc_t __attribute__((ext_vector_type(4)));
  typedef double vec_t __attribute__((ext_vector_type(2)));
  static __device__ __forceinline__ acc_t mma(double a, double b, acc_t c) {
    return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ int row(int i, int g) { return g + 4 * i; }
};

template <typename T>
__device__ __forceinline__ T group_max(T x) {
  constexpr int G = AM<T>::G;
  x = fmax(x, __shfl_xor(x, 32, 64));
  if (G == 4) x = fmax(x, __shfl_xor(x, 16, 64));
  return x;
}
template <typename T>
__device__ __forceinline__ T group_sum(T x) {
  constexpr int G = AM<T>::G;
  x += __shfl_xor(x, 32, 64);
  if (G == 4) x += __shfl_xor(x, 16, 64);
  return x;
}

struct Strides3 {
  int64_t b, h, t;
};

struct AttnArgs {
  const void *q, *k, *v, *o, *dO;
  void *out, *dq, *dk, *dv;
  void *rowmax, *rowsum;  // [B, H, T]
  const void* drow;       // [B, H, T] rowsum(dO * O)
  void* ds;               // [B, H, T, T] dS written by the key-block pass for the dQ pass (or NULL)
  Strides3 sq, sk, sv, so, sdo, sdq, sdk, sdv;
  int64_t B, H, T, D;
  double scale;
  int vec;   // 16-byte global access allowed for every operand
  int ovec;  // the results (out, or dq, dk and dv) too, with D a multiple of the vector
};

// Load NR rows [r0, r0 + NR) of a (T x D) matrix with row stride `rs` into LDS
// [NR][DP + PAD]; rows >= T and columns >= D read as 0.
template <typename T, int NR, int DP>
__device__ __forceinline__ void load_rows(T* __restrict__ lds, const T* __restrict__ base, int64_t rs, int64_t r0,
                                          int64_t Tn, int64_t D, bool vec) {
  constexpr int VEC = AM<T>::VEC, LD = DP + AM<T>::PAD;
  if (vec) {
    constexpr int NV = NR * DP / VEC;
    for (int f = threadIdx.x; f < NV; f += 256) {
      const int r = f / (DP / VEC), d = (f % (DP / VEC)) * VEC;
      typename AM<T>::vec_t x = typename AM<T>::vec_t(0);
      if (r0 + r < Tn && d < D) x = *reinterpret_cast<const typename AM<T>::vec_t*>(base + (r0 + r) * rs + d);
      *reinterpret_cast<typename AM<T>::vec_t*>(lds + r * LD + d) = x;
    }
  } else {
    for (int f = threadIdx.x; f < NR * DP; f += 256) {
      const int r = f / DP, d = f % DP;
      lds[r * LD + d] = (r0 + r < Tn && d < D) ? base[(r0 + r) * rs + d] : T(0);
    }
  }
}

// s_waitcnt vmcnt(0): drain this wave's outstanding global loads. Placed
// before a loop whose body first reads registers loaded ahead of it, so that
// the wait is paid once there and not, at the loop's first use of them, on
// every iteration (the wait analysis merges the loop entry into the loop head).
__device__ __forceinline__ void drain_vm() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// A lane's VEC-vectors of one row (its column c of the wave tile), d-chunked:
// element s of vector ch is d = 8*ch + VEC*g + s.
template <typename T, int DP>
__device__ __forceinline__ void load_frag_rows(typename AM<T>::vec_t (&f)[DP / 8], const T* __restrict__ base,
                                               int64_t rs, int64_t r, int64_t Tn, int64_t D, int g, bool vec) {
  constexpr int VEC = AM<T>::VEC;
  typedef typename AM<T>::vec_t VT;
  if (vec) {
    // every vector load is issued before the first is used: a row past T or
    // a chunk past D reads a valid address and is zeroed afterwards (a load
    // behind a per-lane branch would wait for the one before it)
    const bool in = r < Tn;
    const T* row = base + (in ? r : 0) * rs;
#pragma unroll
    for (int ch = 0; ch < DP / 8; ++ch) {
      const int d = 8 * ch + VEC * g;
      const VT x = *reinterpret_cast<const VT*>(row + (d < D ? d : 0));
      f[ch] = in && d < D ? x : VT(0);
    }
    return;
  }
#pragma unroll
  for (int ch = 0; ch < DP / 8; ++ch) {
    const int d = 8 * ch + VEC * g;
    VT x = VT(0);
    if (r < Tn) {
#pragma unroll
      for (int s = 0; s < VEC; ++s)
        if (d + s < D) x[s] = base[r * rs + d + s];
    }
    f[ch] = x;
  }
}

// acc (MT x MT, rows = LDS rows rbase.., cols = lane's fragment rows) +=
// sum_d lds[rbase + row][d] * frag[col][d]
template <typename T, int DP>
__device__ __forceinline__ typename AM<T>::acc_t mma_rows_frag(typename AM<T>::acc_t acc, const T* __restrict__ lds,
                                                                int rbase, const typename AM<T>::vec_t (&f)[DP / 8],
                                                                int g, int c) {
  constexpr int VEC = AM<T>::VEC, LD = DP + AM<T>::PAD;
#pragma unroll
  for (int ch = 0; ch < DP / 8; ++ch) {
    const typename AM<T>::vec_t a =
        *reinterpret_cast<const typename AM<T>::vec_t*>(lds + (rbase + c) * LD + 8 * ch + VEC * g);
#pragma unroll
    for (int s = 0; s < VEC; ++s) acc = AM<T>::mma(a[s], f[ch][s], acc);
  }
  return acc;
}

// The same product with the B rows also read from LDS: acc += sum_d
// ldsA[rbase + row][d] * ldsB[col][d] (lane column c reads row c of ldsB).
template <typename T, int DP>
__device__ __forceinline__ typename AM<T>::acc_t mma_rows_rows(typename AM<T>::acc_t acc, const T* __restrict__ ldsA,
                                                                const T* __restrict__ ldsB, int g, int c) {
  constexpr int VEC = AM<T>::VEC, LD = DP + AM<T>::PAD;
#pragma unroll
  for (int ch = 0; ch < DP / 8; ++ch) {
    const typename AM<T>::vec_t x = *reinterpret_cast<const typename AM<T>::vec_t*>(ldsA + c * LD + 8 * ch + VEC * g);
    const typename AM<T>::vec_t y = *reinterpret_cast<const typename AM<T>::vec_t*>(ldsB + c * LD + 8 * ch + VEC * g);
#pragma unroll
    for (int s = 0; s < VEC; ++s) acc = AM<T>::mma(x[s], y[s], acc);
  }
  return acc;
}

// out^T (DP x MT, DP/MT tiles over d) += sum_j lds[jbase + j][d] * P(col, j),
// where P for k-slot g at step i is register i of pacc (rows j = row(i, g)).
template <typename T, int DP>
__device__ __forceinline__ void mma_lds_t_regs(typename AM<T>::acc_t (&out)[DP / AM<T>::MT],
                                               const T* __restrict__ lds, int jbase,
                                               const typename AM<T>::acc_t& pacc, int g, int c) {
  constexpr int MT = AM<T>::MT, NACC = AM<T>::NACC, LD = DP + AM<T>::PAD;
#pragma unroll
  for (int i = 0; i < NACC; ++i) {
    const T* rowp = lds + (jbase + AM<T>::row(i, g)) * LD + c;
#pragma unroll
    for (int dt = 0; dt < DP / MT; ++dt) out[dt] = AM<T>::mma(rowp[dt * MT], pacc[i], out[dt]);
  }
}

// Base-2 exponential: one v_exp_f32 for float (softmax probabilities need
// about 1 ulp, which it gives); the accurate library exp2 for double.
__device__ __forceinline__ float ex2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ double ex2(double x) { return exp2(x); }

// Largest excess (log2 units) of a score over the forward's reference max
// before the reference moves: probabilities stay <= 2^8.
constexpr float kLazyLog2 = 8.0f;

// Column swizzle of the transposed LDS tiles: XOR of bits 2-3 of the column
// with bits 4-5 of the row, so groups of 4 columns stay 16-byte aligned and a
// wave's transposed stores (16 rows 4 apart, 4 columns) hit 64 distinct banks.
__device__ __forceinline__ int tswz(int row) { return ((row >> 4) & 3) << 2; }

// Registers for one NR x DP tile in flight from global memory (16-byte
// vectors, 256 threads), stored to LDS [NR][DP + PAD] after the current tile's
// MFMAs. Rows >= Tn and columns >= D are zero.
//
// FAST (16-byte access allowed, D == DP and T a multiple of 128, so every
// tile and every block lies inside [0, T)): every thread issues the same
// loads from persistent pointers with no branch. Otherwise each element is
// bounds-checked.
template <typename T, int NR, int DP, bool FAST>
struct TileFetch {
  typedef typename AM<T>::vec_t V;
  static constexpr int VEC = AM<T>::VEC, LD = DP + AM<T>::PAD;
  static constexpr int TOTAL = NR * DP / VEC;
  static constexpr int NV = (TOTAL + 255) / 256;
  V r[NV];
  // FAST: per-thread source pointers, advanced one tile per next(); kept in
  // registers for the whole loop, so no load address is a temporary that the
  // compiler could hand to an MFMA result while the load is in flight (which
  // makes it wait for every outstanding load first)
  const T* p[NV];
  int64_t step = 0;
  const T* base_ = nullptr;
  int64_t rs_ = 0;
  int r0_ = 0, tn_ = 0, d_ = 0;
  bool vec_ = false;

  // tiles are then fetched at rows r0, r0 + NR, r0 + 2 NR, ...
  __device__ __forceinline__ void start(const T* __restrict__ base, int64_t rs, int r0, int Tn, int D, bool vec) {
    base_ = base;
    rs_ = rs;
    r0_ = r0;
    tn_ = Tn;
    d_ = D;
    vec_ = vec;
    if (FAST) {
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        int f = threadIdx.x + 256 * i;
        if (TOTAL % 256 != 0) f = f < TOTAL ? f : TOTAL - 1;
        const int rr = f / (DP / VEC), d = (f % (DP / VEC)) * VEC;
        p[i] = base + (int64_t)(r0 + rr) * rs + d;
      }
      step = (int64_t)NR * rs;
    }
  }

  // Load the next tile (FAST: every row is inside [0, Tn), the caller's contract).
  __device__ __forceinline__ void next() {
    if (FAST) {
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        r[i] = *reinterpret_cast<const V*>(p[i]);
        p[i] += step;
      }
    } else {
      fetch(base_, rs_, r0_, tn_, d_, vec_);
    }
    r0_ += NR;
  }

  // bounds-checked load of the tile at rows [r0, r0 + NR)
  __device__ __forceinline__ void fetch(const T* __restrict__ base, int64_t rs, int r0, int Tn, int D, bool vec) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int f = threadIdx.x + 256 * i;
      if (TOTAL % 256 != 0 && f >= TOTAL) continue;
      const int rr = f / (DP / VEC), d = (f % (DP / VEC)) * VEC;
      const T* src = base + (int64_t)(r0 + rr) * rs + d;
      if (vec) {
        r[i] = (r0 + rr < Tn && d < D) ? *reinterpret_cast<const V*>(src) : V(0);
      } else {
        V x = V(0);
#pragma unroll
        for (int e = 0; e < VEC; ++e)
          if (r0 + rr < Tn && d + e < D) x[e] = src[e];
        r[i] = x;
      }
    }
  }

  __device__ __forceinline__ V value(int i, int) const { return r[i]; }

  __device__ __forceinline__ void store(T* __restrict__ lds) const {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int f = threadIdx.x + 256 * i;
      if (TOTAL % 256 != 0 && f >= TOTAL) continue;
      const int rr = f / (DP / VEC), d = (f % (DP / VEC)) * VEC;
      *reinterpret_cast<V*>(lds + rr * LD + d) = value(i, rr);
    }
  }

  // The same tile transposed: ldsT[d][row ^ tswz(d)], row stride NR + 4
  // (keeps 16-byte alignment for the vector reads of mma_ldsT_regs; the
  // swizzle spreads a wave's scalar stores over all banks).
  static constexpr int LDT = NR + 4;
  __device__ __forceinline__ void store_t(T* __restrict__ ldsT) const {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int f = threadIdx.x + 256 * i;
      if (TOTAL % 256 != 0 && f >= TOTAL) continue;
      const int rr = f / (DP / VEC), d = (f % (DP / VEC)) * VEC;
      const V x = value(i, rr);
#pragma unroll
      for (int e = 0; e < VEC; ++e) ldsT[(d + e) * LDT + (rr ^ tswz(d + e))] = x[e];
    }
  }
};

// float32 form of mma_lds_t_regs reading a transposed tile ldsT[d][j] (row
// stride LDT): MFMA steps i = 4a .. 4a+3 of lane group g use rows
// j = 8a + 4g + 0..3, four consecutive floats, so one 16-byte read feeds four
// MFMAs instead of one scalar read per MFMA.
template <int DP, int LDT>
__device__ __forceinline__ void mma_ldsT_regs(AM<float>::acc_t (&out)[DP / 32], const float* __restrict__ ldsT,
                                              int jbase, const AM<float>::acc_t& pacc, int g, int c) {
#pragma unroll
  for (int a4 = 0; a4 < 4; ++a4)
#pragma unroll
    for (int dt = 0; dt < DP / 32; ++dt) {
      const int row = dt * 32 + c;
      const AM<float>::vec_t v =
          *reinterpret_cast<const AM<float>::vec_t*>(ldsT + row * LDT + ((jbase + 8 * a4 + 4 * g) ^ tswz(row)));
#pragma unroll
      for (int e = 0; e < 4; ++e) out[dt] = AM<float>::mma(v[e], pacc[4 * a4 + e], out[dt]);
    }
}

// Write a wave's MT x DP result (held transposed: lane column c = row of the
// result, register rows = d) through LDS to global rows r0 + (0 .. NROWS).
// ovec (D == DP, dst and rs 16-byte granular): whole vectors out of LDS and
// to global memory; in float32 a lane's four consecutive rows i = 4a .. 4a+3
// go to LDS as one vector too.
template <typename T, int DP, int NROWS>
__device__ __forceinline__ void store_result(T* __restrict__ lds, const typename AM<T>::acc_t (&acc)[DP / AM<T>::MT],
                                             T mul, T* __restrict__ dst, int64_t rs, int r0, int Tn, int D, int wave,
                                             int g, int c, bool ovec) {
  using M = AM<T>;
  typedef typename M::vec_t V;
  constexpr int MT = M::MT, NACC = M::NACC, LD = DP + M::PAD, VEC = M::VEC;
  T* Ws = lds + wave * MT * LD;
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int dt = 0; dt < DP / MT; ++dt)
#pragma unroll
      for (int a4 = 0; a4 < NACC / 4; ++a4) {
        V x;
#pragma unroll
        for (int e = 0; e < 4; ++e) x[e] = acc[dt][4 * a4 + e] * mul;
        *reinterpret_cast<V*>(Ws + c * LD + dt * MT + M::row(4 * a4, g)) = x;
      }
  } else {
#pragma unroll
    for (int dt = 0; dt < DP / MT; ++dt)
#pragma unroll
      for (int i = 0; i < NACC; ++i) Ws[c * LD + dt * MT + M::row(i, g)] = acc[dt][i] * mul;
  }
  __syncthreads();
  if (ovec) {
    for (int f = threadIdx.x; f < NROWS * DP / VEC; f += 256) {
      const int r = f / (DP / VEC), d = (f % (DP / VEC)) * VEC;
      if (r0 + r < Tn)
        *reinterpret_cast<V*>(dst + (int64_t)(r0 + r) * rs + d) = *reinterpret_cast<const V*>(lds + r * LD + d);
    }
    return;
  }
  for (int f = threadIdx.x; f < NROWS * DP; f += 256) {
    const int r = f / DP, d = f % DP;
    if (r0 + r < Tn && d < D) dst[(int64_t)(r0 + r) * rs + d] = lds[r * LD + d];
  }
}

// ----------------------------------------------------------------- forward
// rowmax is kept in base-2 units: m = log2(e) * max_j (q . k_j * scale).
// Blocks start in linear-id order and are dealt to the 8 XCDs round-robin.
// Causal blocks differ in length (the last query block visits every key
// tile, the first one a single tile), and a long block that starts late
// leaves most of the chip idle while it finishes. So the linear id is split
// as rank * (B*H) + bh: all (batch, head) pairs' longest blocks (rank 0)
// start first, then rank 1, ... With B*H a multiple of 8 every block of one
// (batch, head) also lands on the same XCD, so its K/V (or Q/dO) rows are
// fetched into one L2.
__device__ __forceinline__ void causal_block(int& rank, int& bh) {
  const int L = (int)blockIdx.x + (int)gridDim.x * (int)blockIdx.y;
  rank = L / (int)gridDim.y;
  bh = L % (int)gridDim.y;
}

template <typename T, int DP, bool FAST>
__global__ void __launch_bounds__(256, 2) attn_fwd_kernel(AttnArgs a) {
  using M = AM<T>;
  constexpr int MT = M::MT, NACC = M::NACC, LD = DP + M::PAD;
  constexpr int KB = 2 * MT;  // keys per tile
  constexpr int QB = 4 * MT;  // queries per block (MT per wave)
  constexpr int TILE = KB * LD, STAGE = 2 * TILE;
  constexpr int LDS_N = 2 * STAGE > QB * LD ? 2 * STAGE : QB * LD;
  __shared__ __attribute__((aligned(16))) T lds[LDS_N];

  int bx, bh;  // bx: length rank (0 = longest)
  causal_block(bx, bh);
  const int64_t b = bh / a.H, h = bh % a.H;
  const int Tn = (int)a.T, D = (int)a.D;
  const int q0 = (int)(gridDim.x - 1 - bx) * QB;  // longest causal rows first
  // the wave index in a scalar register: conditions on it are wave-uniform branches
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane / MT, c = lane % MT;
  const int wq0 = q0 + wave * MT;
  const int qr = wq0 + c;  // this lane's query (column)
  const T* Q = (const T*)a.q + b * a.sq.b + h * a.sq.h;
  const T* K = (const T*)a.k + b * a.sk.b + h * a.sk.h;
  const T* V = (const T*)a.v + b * a.sv.b + h * a.sv.h;
  const T sl2 = (T)(a.scale * 1.4426950408889634);  // scale * log2(e)
  const T ninf = -INFINITY;
  const bool vec = a.vec != 0;

  typename M::vec_t qf[DP / 8];
  load_frag_rows<T, DP>(qf, Q, a.sq.t, qr, Tn, D, g, vec);
  if constexpr (FAST && sizeof(T) == 4) {
    // scores straight in base-2 units: q * scale * log2(e) once, not per score
#pragma unroll
    for (int ch = 0; ch < DP / 8; ++ch) qf[ch] *= sl2;
  }
  typename M::acc_t oacc[DP / MT];
#pragma unroll
  for (int dt = 0; dt < DP / MT; ++dt) oacc[dt] = typename M::acc_t(0);
  T mrow = ninf, lrow = T(0);
  constexpr bool LAZY = FAST && sizeof(T) == 4;
  T mtop = ninf;  // LAZY: this lane's running max of its own scores

  const int qlast = (q0 + QB < Tn ? q0 + QB : Tn) - 1;
  const int nkb = qlast / KB + 1;
  TileFetch<T, KB, DP, FAST> fk, fv;
  fk.start(K, a.sk.t, 0, Tn, D, vec);
  fv.start(V, a.sv.t, 0, Tn, D, vec);
  fk.next();
  fv.next();
  fk.store(lds);
  fv.store(lds + TILE);
  __syncthreads();
  for (int kb = 0; kb < nkb; ++kb) {
    const int k0 = kb * KB;
    const T* Ks = lds + (kb & 1) * STAGE;
    const T* Vs = Ks + TILE;
    const bool more = kb + 1 < nkb;
    if (more) {
      fk.next();
      fv.next();
    }
    // a wave whose queries all precede the tile's keys has nothing to add (all
    // its probabilities would be 0 and its max/sum unchanged): skip the work
    if (k0 <= wq0 + MT - 1) {
      typename M::acc_t sacc[KB / MT];
#pragma unroll
      for (int jt = 0; jt < KB / MT; ++jt) sacc[jt] = mma_rows_frag<T, DP>(typename M::acc_t(0), Ks, jt * MT, qf, g, c);
      // causal mask only where a key of the tile can exceed a query of the wave
      const bool mask = (k0 + KB - 1 > wq0) || (k0 + KB > Tn);
      T bmax = ninf;
      // the mask test hoisted out of the per-score loop (two copies of it)
      auto scores = [&](auto maskc) {
        constexpr bool MASK = decltype(maskc)::value;
#pragma unroll
        for (int jt = 0; jt < KB / MT; ++jt)
#pragma unroll
          for (int i = 0; i < NACC; ++i) {
            T s = FAST && sizeof(T) == 4 ? sacc[jt][i] : sacc[jt][i] * sl2;
            if constexpr (MASK) {
              const int j = k0 + jt * MT + M::row(i, g);
              s = (j <= qr && j < Tn) ? s : ninf;
            }
            sacc[jt][i] = s;
            bmax = fmax(bmax, s);
          }
      };
      if (mask)
        scores(std::true_type());
      else
        scores(std::false_type());
      if constexpr (LAZY) {
        // Lazy rescaling: the probabilities are taken against a reference
        // max mrow (equal across the lane groups of a query column) that
        // moves only when a score exceeds it by more than kLazyLog2, so
        // p <= 2^kLazyLog2 and the output and sum are rescaled a few times
        // per row instead of on almost every tile; no cross-lane step on the
        // other tiles. The row sum stays a per-lane partial until the end.
        // The first tile a wave computes holds key 0 for every query, so
        // mrow is finite after it.
        mtop = fmax(mtop, bmax);
        if (__any(bmax > mrow + kLazyLog2)) {
          const T mnew = fmax(mrow, group_max(bmax));
          const T alpha = ex2(mrow - mnew);  // mrow = -inf on the first tile: 0
          lrow *= alpha;
#pragma unroll
          for (int dt = 0; dt < DP / MT; ++dt) oacc[dt] *= alpha;
          mrow = mnew;
        }
#pragma unroll
        for (int jt = 0; jt < KB / MT; ++jt)
#pragma unroll
          for (int i = 0; i < NACC; ++i) {
            const T p = ex2(sacc[jt][i] - mrow);
            sacc[jt][i] = p;
            lrow += p;
          }
      } else {
        bmax = group_max(bmax);
        const T mnew = fmax(mrow, bmax);
        // aligned path: every query sees key 0 in the first tile, so the max is
        // finite from then on
        const bool live = FAST || mnew != ninf;
        const T alpha = live ? ex2(mrow - mnew) : T(1);
        T psum = T(0);
#pragma unroll
        for (int jt = 0; jt < KB / MT; ++jt)
#pragma unroll
          for (int i = 0; i < NACC; ++i) {
            const T p = live ? ex2(sacc[jt][i] - mnew) : T(0);
            sacc[jt][i] = p;
            psum += p;
          }
        psum = group_sum(psum);
        lrow = lrow * alpha + psum;
        mrow = mnew;
        // rescale the output only when some lane's max moved (alpha == 1
        // leaves it unchanged bit for bit)
        if (__any(alpha != T(1))) {
#pragma unroll
          for (int dt = 0; dt < DP / MT; ++dt) oacc[dt] *= alpha;
        }
      }
#pragma unroll
      for (int jt = 0; jt < KB / MT; ++jt) mma_lds_t_regs<T, DP>(oacc, Vs, jt * MT, sacc[jt], g, c);
    }
    if (more) {
      T* nxt = lds + ((kb + 1) & 1) * STAGE;
      fk.store(nxt);
      fv.store(nxt + TILE);
    }
    __syncthreads();
  }
  if constexpr (LAZY) {
    // the row's sum against the reference max, then (after the output) the
    // statistics against the true max
    lrow = group_sum(lrow);
    mtop = group_max(mtop);
  }
  T* O = (T*)a.out + b * a.so.b + h * a.so.h;
  store_result<T, DP, QB>(lds, oacc, lrow > T(0) ? T(1) / lrow : T(0), O, a.so.t, q0, Tn, D, wave, g, c,
                          a.ovec != 0 && D == DP);
  if constexpr (LAZY) {
    lrow *= ex2(mrow - mtop);
    mrow = mtop;
  }
  if (g == 0 && qr < Tn) {
    ((T*)a.rowmax)[(int64_t)bh * Tn + qr] = mrow;
    ((T*)a.rowsum)[(int64_t)bh * Tn + qr] = lrow;
  }
}

// D_r = sum_d dO[r, d] * O[r, d]  (= rowsum(dP * P), the softmax-backward term)
template <typename T>
__global__ void __launch_bounds__(256) attn_drow_kernel(AttnArgs a) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t total = a.B * a.H * a.T;
  if (row >= total) return;
  const int64_t t = row % a.T, bh = row / a.T, b = bh / a.H, h = bh % a.H;
  const T* O = (const T*)a.o + b * a.so.b + h * a.so.h + t * a.so.t;
  const T* G = (const T*)a.dO + b * a.sdo.b + h * a.sdo.h + t * a.sdo.t;
  T s = T(0);
  for (int64_t d = lane; d < a.D; d += 64) s += O[d] * G[d];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
  if (lane == 0) ((T*)a.drow)[row] = s;
}

// Rows of D = 64: 16 lanes per row, four consecutive elements of O and dO
// each (one 16-byte vector in float32, two in float64), two rows per lane
// group (both rows' loads in flight at once), 32 rows per 256-thread block.
template <typename T>
__global__ void __launch_bounds__(256) attn_drow64_kernel(AttnArgs a) {
  typedef T v4 __attribute__((ext_vector_type(4)));
  constexpr int RPT = 2;
  const int q = threadIdx.x & 15;
  const int64_t total = a.B * a.H * a.T;
  const int64_t row0 = ((int64_t)blockIdx.x * 16 + (threadIdx.x >> 4)) * RPT;
  v4 o[RPT], g[RPT];
#pragma unroll
  for (int u = 0; u < RPT; ++u) {
    const int64_t row = row0 + u;
    o[u] = g[u] = v4(0);
    if (row < total) {
      const int64_t t = row % a.T, bh = row / a.T, b = bh / a.H, h = bh % a.H;
      o[u] = *reinterpret_cast<const v4*>((const T*)a.o + b * a.so.b + h * a.so.h + t * a.so.t + 4 * q);
      g[u] = *reinterpret_cast<const v4*>((const T*)a.dO + b * a.sdo.b + h * a.sdo.h + t * a.sdo.t + 4 * q);
    }
  }
#pragma unroll
  for (int u = 0; u < RPT; ++u) {
    T s = ((o[u][0] * g[u][0] + o[u][1] * g[u][1]) + o[u][2] * g[u][2]) + o[u][3] * g[u][3];
#pragma unroll
    for (int off = 8; off >= 1; off >>= 1) s += __shfl_xor(s, off, 16);
    if (q == 0 && row0 + u < total) ((T*)a.drow)[row0 + u] = s;
  }
}

// ------------------------------------------------- backward A: dK and dV
// One block owns 4*MT keys (MT per wave, as the columns of its tiles) and walks
// the query tiles of MT rows that can see them, double-buffered.
template <typename T, int DP, bool FAST>
__global__ void __launch_bounds__(256, 2) attn_bwd_kv_kernel(AttnArgs a) {
  using M = AM<T>;
  constexpr int MT = M::MT, NACC = M::NACC, LD = DP + M::PAD;
  constexpr bool F32 = sizeof(T) == 4;
  constexpr int QT = MT;      // queries per tile
  constexpr int KBB = 4 * MT;  // keys per block
  constexpr int LDT = QT + 4;  // transposed tiles (float32): [DP][QT + 4]
  constexpr int TILE = QT * LD, TILE_T = F32 ? DP * LDT : 0;
  constexpr int STAGE = 2 * TILE + 2 * TILE_T;  // Q, dO (+ their transposes)
  constexpr int LDS_N = 2 * STAGE > KBB * LD ? 2 * STAGE : KBB * LD;
  __shared__ __attribute__((aligned(16))) T lds[LDS_N];
  // per query row: max (base 2), 1 / sum, rowsum(dO * O), max + log2(sum)
  __shared__ __attribute__((aligned(16))) T stats[2][4][QT];

  int bx, bh;  // bx: length rank (0 = longest)
  causal_block(bx, bh);
  const int64_t b = bh / a.H, h = bh % a.H;
  const int Tn = (int)a.T, D = (int)a.D;
  const int k0 = bx * KBB;
  // the wave index in a scalar register: conditions on it are wave-uniform branches
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane / MT, c = lane % MT;
  const int wk0 = k0 + wave * MT;
  const int kj = wk0 + c;  // this lane's key (column)
  const T* Q = (const T*)a.q + b * a.sq.b + h * a.sq.h;
  const T* K = (const T*)a.k + b * a.sk.b + h * a.sk.h;
  const T* V = (const T*)a.v + b * a.sv.b + h * a.sv.h;
  const T* G = (const T*)a.dO + b * a.sdo.b + h * a.sdo.h;
  const T* RM = (const T*)a.rowmax + (int64_t)bh * Tn;
  const T* RS = (const T*)a.rowsum + (int64_t)bh * Tn;
  const T* DR = (const T*)a.drow + (int64_t)bh * Tn;
  T* DS = a.ds ? (T*)a.ds + (int64_t)bh * Tn * Tn : nullptr;
  const T sl2 = (T)(a.scale * 1.4426950408889634);
  const bool vec = a.vec != 0;
  // this lane's dS byte offset from a tile's first row: row 4g (float32) or g
  // (float64), column kj
  const unsigned ds_lane = (unsigned)((F32 ? 4 * g : g) * Tn + kj) * (unsigned)sizeof(T);

  typename M::vec_t kf[DP / 8], vf[DP / 8];
  load_frag_rows<T, DP>(kf, K, a.sk.t, kj, Tn, D, g, vec);
  load_frag_rows<T, DP>(vf, V, a.sv.t, kj, Tn, D, g, vec);
  typename M::acc_t dk[DP / MT], dv[DP / MT];
#pragma unroll
  for (int dt = 0; dt < DP / MT; ++dt) dk[dt] = dv[dt] = typename M::acc_t(0);

  const int qs0 = (k0 / QT) * QT;
  const int nqt = k0 < Tn ? (Tn - qs0 + QT - 1) / QT : 0;
  TileFetch<T, QT, DP, FAST> fq, fg;
  T st0 = T(0), st1 = T(1), st2 = T(0);
  // FAST: every thread loads (lanes past QT re-read a valid row; only the
  // first QT threads store), from pointers advanced one tile per call
  const int srow = qs0 + (int)(threadIdx.x % QT);
  const T *rm_p = RM + srow, *rs_p = RS + srow, *dr_p = DR + srow;
  auto fetch_stats = [&](int qs) {
    if (FAST) {
      st0 = *rm_p;
      st1 = *rs_p;
      st2 = *dr_p;
      rm_p += QT;
      rs_p += QT;
      dr_p += QT;
    } else if (threadIdx.x < QT) {
      const int r = qs + threadIdx.x;
      const bool ok = r < Tn;
      st0 = ok ? RM[r] : T(0);
      st1 = ok ? RS[r] : T(1);
      st2 = ok ? DR[r] : T(0);
    }
  };
  auto store_stage = [&](int stage) {
    T* base = lds + stage * STAGE;
    fq.store(base);
    fg.store(base + TILE);
    if constexpr (F32) {
      fq.store_t(base + 2 * TILE);
      fg.store_t(base + 2 * TILE + TILE_T);
    }
    if (threadIdx.x < QT) {  // the loads were issued a tile earlier; 1 / sum only now, after the MFMAs
      stats[stage][0][threadIdx.x] = st0;
      stats[stage][1][threadIdx.x] = T(1) / st1;
      stats[stage][2][threadIdx.x] = st2;
      stats[stage][3][threadIdx.x] = st0 + log2(st1);
    }
  };
  if (nqt > 0) {
    fq.start(Q, a.sq.t, qs0, Tn, D, vec);
    fg.start(G, a.sdo.t, qs0, Tn, D, vec);
    fq.next();
    fg.next();
    fetch_stats(qs0);
    store_stage(0);
  }
  drain_vm();
  __syncthreads();
  for (int it = 0; it < nqt; ++it) {
    const int qs = qs0 + it * QT;
    const int cur = it & 1;
    const T* Qs = lds + cur * STAGE;
    const T* Gs = Qs + TILE;
    const bool more = it + 1 < nqt;
    if (more) {
      fq.next();
      fg.next();
      fetch_stats(qs + QT);
    }
    // a tile whose queries all precede this wave's keys contributes nothing
    // (and its dS is never read): skip it
    if (qs + QT - 1 >= wk0) {
      // S(r, j) and dP(r, j): rows r = the tile's queries (LDS), columns j = this wave's keys
      typename M::acc_t s = mma_rows_frag<T, DP>(typename M::acc_t(0), Qs, 0, kf, g, c);
      typename M::acc_t dp = mma_rows_frag<T, DP>(typename M::acc_t(0), Gs, 0, vf, g, c);
      const bool mask = (qs < wk0 + MT - 1) || (qs + QT > Tn) || (wk0 + MT > Tn);
      auto prob = [&](int i, T m, T linv, T dr) {
        T p = ex2(s[i] * sl2 - m) * linv;
        if (mask) {
          const int r = qs + M::row(i, g);
          p = (kj <= r && r < Tn && kj < Tn) ? p : T(0);
        }
        s[i] = p;
        dp[i] = p * (dp[i] - dr);
        if (DS) {
          const int r = qs + M::row(i, g);
          if (r < Tn && kj < Tn) DS[(int64_t)r * Tn + kj] = dp[i];
        }
      };
      if constexpr (F32) {
        if constexpr (FAST) {
          // Every row of the tile and every key of the block lie inside
          // [0, T): no bounds tests. P = 2^(s sl2 - (m + log2 sum)): one
          // fma and one exp. dS rows are addressed from a wave-uniform row
          // pointer plus this lane's fixed offset, so the stores take no
          // vector address arithmetic.
          const int lim = kj - qs - 4 * g;  // row qs + 4g + x sees key kj iff x >= lim
          T* dsb = DS + (int64_t)qs * Tn;  // the aligned path always runs with the dS workspace
          // the mask test hoisted out of the per-score loop
          auto probs = [&](auto maskc) {
            constexpr bool MASK = decltype(maskc)::value;
#pragma unroll
            for (int a4 = 0; a4 < NACC / 4; ++a4) {
              const int r0 = 8 * a4 + 4 * g;
              const typename M::vec_t ml4 = *reinterpret_cast<const typename M::vec_t*>(&stats[cur][3][r0]);
              const typename M::vec_t d4 = *reinterpret_cast<const typename M::vec_t*>(&stats[cur][2][r0]);
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const int i = 4 * a4 + e;
                T p = ex2(__builtin_fmaf(s[i], sl2, -ml4[e]));
                if constexpr (MASK) p = 8 * a4 + e >= lim ? p : T(0);
                s[i] = p;
                const T v = p * (dp[i] - d4[e]);
                dp[i] = v;
                *(T*)((char*)(dsb + (int64_t)(8 * a4 + e) * Tn) + ds_lane) = v;
              }
            }
          };
          if (mask)
            probs(std::true_type());
          else
            probs(std::false_type());
        } else {
          // rows 8a + 4g + 0..3 of MFMA steps 4a .. 4a+3: one 16-byte read per statistic
#pragma unroll
          for (int a4 = 0; a4 < NACC / 4; ++a4) {
            const int r0 = 8 * a4 + 4 * g;
            const typename M::vec_t m4 = *reinterpret_cast<const typename M::vec_t*>(&stats[cur][0][r0]);
            const typename M::vec_t l4 = *reinterpret_cast<const typename M::vec_t*>(&stats[cur][1][r0]);
            const typename M::vec_t d4 = *reinterpret_cast<const typename M::vec_t*>(&stats[cur][2][r0]);
#pragma unroll
            for (int e = 0; e < 4; ++e) prob(4 * a4 + e, m4[e], l4[e], d4[e]);
          }
        }
        // dV^T += dO^T P ; dK^T += Q^T dS (transposed tiles: vector reads)
        mma_ldsT_regs<DP, LDT>(dv, Qs + 2 * TILE + TILE_T, 0, s, g, c);
        mma_ldsT_regs<DP, LDT>(dk, Qs + 2 * TILE, 0, dp, g, c);
      } else {
        if constexpr (FAST) {
          // Every row of the tile and every key of the block lie inside
          // [0, T): no bounds tests; dS rows qs + g + 4i are addressed from a
          // wave-uniform row pointer plus this lane's fixed offset, so the
          // stores take no vector address arithmetic (same values as prob).
          T* dsb = DS + (int64_t)qs * Tn;
          auto probs = [&](auto maskc) {
            constexpr bool MASK = decltype(maskc)::value;
#pragma unroll
            for (int i = 0; i < NACC; ++i) {
              const int rl = M::row(i, g);
              T p = ex2(s[i] * sl2 - stats[cur][0][rl]) * stats[cur][1][rl];
              if constexpr (MASK) p = kj <= qs + rl ? p : T(0);
              s[i] = p;
              const T v = p * (dp[i] - stats[cur][2][rl]);
              dp[i] = v;
              *(T*)((char*)(dsb + (int64_t)(4 * i) * Tn) + ds_lane) = v;
            }
          };
          if (mask)
            probs(std::true_type());
          else
            probs(std::false_type());
        } else {
#pragma unroll
          for (int i = 0; i < NACC; ++i) {
            const int rl = M::row(i, g);
            prob(i, stats[cur][0][rl], stats[cur][1][rl], stats[cur][2][rl]);
          }
        }
        mma_lds_t_regs<T, DP>(dv, Gs, 0, s, g, c);
        mma_lds_t_regs<T, DP>(dk, Qs, 0, dp, g, c);
      }
    }
    if (more) store_stage(cur ^ 1);
    __syncthreads();
  }
  T* DK = (T*)a.dk + b * a.sdk.b + h * a.sdk.h;
  T* DV = (T*)a.dv + b * a.sdv.b + h * a.sdv.h;
  const bool ovec = a.ovec != 0 && D == DP;
  store_result<T, DP, KBB>(lds, dk, (T)a.scale, DK, a.sdk.t, k0, Tn, D, wave, g, c, ovec);
  __syncthreads();
  store_result<T, DP, KBB>(lds, dv, T(1), DV, a.sdv.t, k0, Tn, D, wave, g, c, ovec);
}

// ------------------------------------------------------- backward B: dQ
// dQ from the dS the key-block pass wrote: dQ^T += K^T dS^T over the key
// tiles up to the block's last query, with dS read straight into the MFMA B
// operand (lane column = query, k-slot = key), so S, P and dP are not
// recomputed. Key tiles wholly above a wave's queries are skipped by that
// wave (their dS is zero).
template <typename T, int DP, bool FAST>
__global__ void __launch_bounds__(256, 2) attn_bwd_q_ds_kernel(AttnArgs a) {
  using M = AM<T>;
  constexpr int MT = M::MT, NACC = M::NACC, LD = DP + M::PAD;
  constexpr bool F32 = sizeof(T) == 4;
  constexpr int KT = MT;      // keys per tile
  constexpr int QB = 4 * MT;  // queries per block
  constexpr int LDT = KT + 4;
  constexpr int TILE = F32 ? DP * LDT : KT * LD;  // K^T [DP][KT + 4] (float32) or K [KT][LD]
  constexpr int LDS_N = 2 * TILE > QB * LD ? 2 * TILE : QB * LD;
  __shared__ __attribute__((aligned(16))) T lds[LDS_N];

  int bx, bh;  // bx: length rank (0 = longest)
  causal_block(bx, bh);
  const int64_t b = bh / a.H, h = bh % a.H;
  const int Tn = (int)a.T, D = (int)a.D;
  const int q0 = (int)(gridDim.x - 1 - bx) * QB;  // longest causal rows first
  // the wave index in a scalar register: conditions on it are wave-uniform branches
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane / MT, c = lane % MT;
  const int wq0 = q0 + wave * MT;
  const int qr = wq0 + c;
  const T* K = (const T*)a.k + b * a.sk.b + h * a.sk.h;
  const T* DS = (const T*)a.ds + (int64_t)bh * Tn * Tn;
  const bool vec = a.vec != 0;
  // float64, aligned: dS through a buffer resource over the (batch, head)
  // block when its byte offsets fit in 32 bits (T <= 23170)
  const bool ds_buf = !F32 && FAST && (uint64_t)Tn * Tn * sizeof(T) <= 0xFFFFFFFFull;
  const Rsrc rS = make_rsrc(DS, (uint64_t)Tn * Tn * sizeof(T));
  const uint32_t ds_lane = ds_buf ? (uint32_t)(((int64_t)qr * Tn + g) * (int64_t)sizeof(T)) : 0u;

  typename M::acc_t dq[DP / MT];
#pragma unroll
  for (int dt = 0; dt < DP / MT; ++dt) dq[dt] = typename M::acc_t(0);

  const int qlast = (q0 + QB < Tn ? q0 + QB : Tn) - 1;
  const int nkt = q0 < Tn ? qlast / KT + 1 : 0;
  auto live = [&](int kt) { return kt * KT <= wq0 + MT - 1 && wq0 < Tn; };
  // lane (c, g), register i: dS[qr][kt * KT + row(i, g)]
  auto load_ds = [&](int kt, typename M::acc_t& r) {
    const int j0 = kt * KT;
    if constexpr (F32 && FAST) {
      // branch-free 16-byte loads (T is a multiple of 4, so a group of four
      // columns is wholly in or out); addresses past the end are clamped and
      // those entries zeroed by valid_ds before use
      const int row = qr < Tn ? qr : Tn - 1;
#pragma unroll
      for (int a4 = 0; a4 < NACC / 4; ++a4) {
        int j = j0 + 8 * a4 + 4 * g;
        j = j + 4 <= Tn ? j : Tn - 4;
        const typename M::vec_t v = *reinterpret_cast<const typename M::vec_t*>(DS + (int64_t)row * Tn + j);
#pragma unroll
        for (int e = 0; e < 4; ++e) r[4 * a4 + e] = v[e];
      }
    } else {
      if constexpr (!F32 && FAST) {
        if (ds_buf) {
          // row qr, columns j0 + g + 4 i (every one inside [0, T) on the
          // aligned path): this lane's byte offset fixed, the tile's and the
          // register's wave-uniform
#pragma unroll
          for (int i = 0; i < NACC; ++i) r[i] = buf_load_f64(rS, ds_lane, (uint32_t)(j0 + 4 * i) * (uint32_t)sizeof(T));
          return;
        }
      }
#pragma unroll
      for (int i = 0; i < NACC; ++i) {
        const int j = j0 + M::row(i, g);
        r[i] = (qr < Tn && j < Tn) ? DS[(int64_t)qr * Tn + j] : T(0);
      }
    }
  };
  auto valid_ds = [&](int kt, typename M::acc_t& r) {
    if constexpr (F32 && FAST) {
#pragma unroll
      for (int i = 0; i < NACC; ++i) {
        const int j = kt * KT + M::row(i, g);
        r[i] = (qr < Tn && j < Tn) ? r[i] : T(0);
      }
    }
  };
  TileFetch<T, KT, DP, FAST> fk;
  auto store_k = [&](int stage) {
    if constexpr (F32)
      fk.store_t(lds + stage * TILE);
    else
      fk.store(lds + stage * TILE);
  };
  typename M::acc_t dsr = typename M::acc_t(0), dsn = typename M::acc_t(0);
  if (nkt > 0) {
    fk.start(K, a.sk.t, 0, Tn, D, vec);
    fk.next();
    store_k(0);
    if (live(0)) load_ds(0, dsr);
  }
  drain_vm();
  __syncthreads();
  for (int kt = 0; kt < nkt; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nkt;
    if (more) {
      fk.next();
      if (live(kt + 1)) load_ds(kt + 1, dsn);
    }
    if (live(kt)) {
      valid_ds(kt, dsr);
      if constexpr (F32)
        mma_ldsT_regs<DP, LDT>(dq, lds + cur * TILE, 0, dsr, g, c);
      else
        mma_lds_t_regs<T, DP>(dq, lds + cur * TILE, 0, dsr, g, c);
    }
    if (more) store_k(cur ^ 1);
    dsr = dsn;
    __syncthreads();
  }
  T* DQ = (T*)a.dq + b * a.sdq.b + h * a.sdq.h;
  store_result<T, DP, QB>(lds, dq, (T)a.scale, DQ, a.sdq.t, q0, Tn, D, wave, g, c, a.ovec != 0 && D == DP);
}

// dQ from the dS workspace, one query tile per block (float32): the block's
// four waves take the key tiles up to the query tile in turn (wave w: tiles
// w, w + 4, ...), each staging its key tile's rows in its own LDS region and
// prefetching the next tile's K rows and dS entries into registers; the four
// partial dQ are added in wave order at the end. Aligned path only (D = DP =
// 64, T a multiple of 32, 16-byte access).
template <typename T, int DP, bool FAST>
__global__ void __launch_bounds__(256, 2) attn_bwd_q_kernel(AttnArgs a) {
  using M = AM<T>;
  constexpr int MT = M::MT, NACC = M::NACC, LD = DP + M::PAD;
  constexpr int KB = 2 * MT;
  constexpr int QB = 4 * MT;
  constexpr int TILE = KB * LD, STAGE = 2 * TILE;
  constexpr int LDS_N = 2 * STAGE > QB * LD ? 2 * STAGE : QB * LD;
  __shared__ __attribute__((aligned(16))) T lds[LDS_N];

  int bx, bh;  // bx: length rank (0 = longest)
  causal_block(bx, bh);
  const int64_t b = bh / a.H, h = bh % a.H;
  const int Tn = (int)a.T, D = (int)a.D;
  const int q0 = (int)(gridDim.x - 1 - bx) * QB;  // longest causal rows first
  // the wave index in a scalar register: conditions on it are wave-uniform branches
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane / MT, c = lane % MT;
  const int wq0 = q0 + wave * MT;
  const int qr = wq0 + c;
  const T* Q = (const T*)a.q + b * a.sq.b + h * a.sq.h;
  const T* K = (const T*)a.k + b * a.sk.b + h * a.sk.h;
  const T* V = (const T*)a.v + b * a.sv.b + h * a.sv.h;
  const T* G = (const T*)a.dO + b * a.sdo.b + h * a.sdo.h;
  const T sl2 = (T)(a.scale * 1.4426950408889634);
  const bool vec = a.vec != 0;
  const bool qok = qr < Tn;
  const T mq = qok ? ((const T*)a.rowmax)[(int64_t)bh * Tn + qr] : T(0);
  const T linv = qok ? T(1) / ((const T*)a.rowsum)[(int64_t)bh * Tn + qr] : T(0);
  const T dq_r = qok ? ((const T*)a.drow)[(int64_t)bh * Tn + qr] : T(0);

  typename M::vec_t qf[DP / 8], gf[DP / 8];
  load_frag_rows<T, DP>(qf, Q, a.sq.t, qr, Tn, D, g, vec);
  load_frag_rows<T, DP>(gf, G, a.sdo.t, qr, Tn, D, g, vec);
  typename M::acc_t dq[DP / MT];
#pragma unroll
  for (int dt = 0; dt < DP / MT; ++dt) dq[dt] = typename M::acc_t(0);

  const int qlast = (q0 + QB < Tn ? q0 + QB : Tn) - 1;
  const int nkb = q0 < Tn ? qlast / KB + 1 : 0;
  TileFetch<T, KB, DP, FAST> fk, fv;
  if (nkb > 0) {
    fk.start(K, a.sk.t, 0, Tn, D, vec);
    fv.start(V, a.sv.t, 0, Tn, D, vec);
    fk.next();
    fv.next();
    fk.store(lds);
    fv.store(lds + TILE);
  }
  __syncthreads();
  for (int kb = 0; kb < nkb; ++kb) {
    const int k0 = kb * KB;
    const T* Ks = lds + (kb & 1) * STAGE;
    const T* Vs = Ks + TILE;
    const bool more = kb + 1 < nkb;
    if (more) {
      fk.next();
      fv.next();
    }
    const bool mask = (k0 + KB - 1 > wq0) || (k0 + KB > Tn) || !qok;
#pragma unroll 1
    for (int jt = 0; jt < KB / MT; ++jt) {
      // S^T(j, r), dP^T(j, r): rows j = keys (LDS), columns r = this wave's queries
      typename M::acc_t s = mma_rows_frag<T, DP>(typename M::acc_t(0), Ks, jt * MT, qf, g, c);
      typename M::acc_t dp = mma_rows_frag<T, DP>(typename M::acc_t(0), Vs, jt * MT, gf, g, c);
#pragma unroll
      for (int i = 0; i < NACC; ++i) {
        T p = ex2(s[i] * sl2 - mq) * linv;
        if (mask) {
          const int j = k0 + jt * MT + M::row(i, g);
          p = (j <= qr && qok && j < Tn) ? p : T(0);
        }
        dp[i] = p * (dp[i] - dq_r);
      }
      // dQ^T += K^T dS^T
      mma_lds_t_regs<T, DP>(dq, Ks, jt * MT, dp, g, c);
    }
    if (more) {
      T* nxt = lds + ((kb + 1) & 1) * STAGE;
      fk.store(nxt);
      fv.store(nxt + TILE);
    }
    __syncthreads();
  }
  T* DQ = (T*)a.dq + b * a.sdq.b + h * a.sdq.h;
  store_result<T, DP, QB>(lds, dq, (T)a.scale, DQ, a.sdq.t, q0, Tn, D, wave, g, c, a.ovec != 0 && D == DP);
}

// ------------------------------------------- head dimensions beyond 64
// For D > 64 the scores of one batch element are materialised, [H, T, T] in
// a pooled workspace, and the products run as batched GEMMs (dtmi_gemm):
// S = Q K^T, P = softmax(S * scale + mask), O = P V; backward P recomputed
// from S and the saved row statistics, dV = P^T dO, dP = dO V^T,
// dS = P * (dP - rowsum(dP * P)) * scale, dQ = dS K, dK = dS^T Q -- dtrain's
// products (autograd.py:226-246), one batch element at a time. One block per
// row for the row passes, fixed reduction order.
// ----------------------------- backward on 16 x 16 tiles over paired ranges
// MFMA 16 x 16 x 4 (float32): lane (g, c), g = lane / 16, supplies column c
// (B operand) or row c (A operand) at k-slot g, and holds column c, rows
// row(i, g) = 4 g + i (i = 0..3) of the 16 x 16 result.
template <typename T>
struct A16;
template <>
struct A16<float> {
  typedef float acc_t __attribute__((ext_vector_type(4)));
  typedef float vec_t __attribute__((ext_vector_type(4)));
  static constexpr int VEC = 4;
  static __device__ __forceinline__ acc_t mma(float a, float b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ int row(int i, int g) { return 4 * g + i; }
};

template <typename VT>
__device__ __forceinline__ VT buf_load_v(Rsrc r, uint32_t voff, uint32_t soff) {
  static_assert(sizeof(VT) == 16, "16-byte vectors");
  return __builtin_bit_cast(VT, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0));
}
// dK (times the softmax scale) and dV of 16 keys from the key pass's
// accumulators: lane (g, c), tile t, register i holds key k0 + c,
// d = 4 row(i, g) + t.
template <typename T>
__device__ __forceinline__ void store_kv16(const AttnArgs& a, int64_t b, int64_t h, int k0,
                                           const typename A16<T>::acc_t (&dk)[4],
                                           const typename A16<T>::acc_t (&dv)[4], int g, int c) {
  using M = A16<T>;
  T* DK = (T*)a.dk + b * a.sdk.b + h * a.sdk.h + (int64_t)(k0 + c) * a.sdk.t;
  T* DV = (T*)a.dv + b * a.sdv.b + h * a.sdv.h + (int64_t)(k0 + c) * a.sdv.t;
  const T scale = (T)a.scale;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = 4 * M::row(i, g);
    const typename M::acc_t xk = {dk[0][i] * scale, dk[1][i] * scale, dk[2][i] * scale, dk[3][i] * scale};
    const typename M::acc_t xv = {dv[0][i], dv[1][i], dv[2][i], dv[3][i]};
    if (a.ovec) {
#pragma unroll
      for (int v = 0; v < 4 / M::VEC; ++v) {
        typename M::vec_t yk, yv;
#pragma unroll
        for (int e = 0; e < M::VEC; ++e) {
          yk[e] = xk[M::VEC * v + e];
          yv[e] = xv[M::VEC * v + e];
        }
        *reinterpret_cast<typename M::vec_t*>(DK + d + M::VEC * v) = yk;
        *reinterpret_cast<typename M::vec_t*>(DV + d + M::VEC * v) = yv;
      }
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        DK[d + t] = xk[t];
        DV[d + t] = xv[t];
      }
    }
  }
}

// dQ (times the softmax scale) of 16 queries from the dQ pass's accumulators:
// lane (g, c), tile t, register i holds row q0 + row(i, g), d = 4 c + t.
template <typename T>
__device__ __forceinline__ void store_q16(const AttnArgs& a, int64_t b, int64_t h, int q0,
                                          const typename A16<T>::acc_t (&dq)[4], int g, int c) {
  using M = A16<T>;
  T* DQ = (T*)a.dq + b * a.sdq.b + h * a.sdq.h + 4 * c;
  const T scale = (T)a.scale;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    T* row = DQ + (int64_t)(q0 + M::row(i, g)) * a.sdq.t;
    const typename M::acc_t x = {dq[0][i] * scale, dq[1][i] * scale, dq[2][i] * scale, dq[3][i] * scale};
    if (a.ovec) {
#pragma unroll
      for (int v = 0; v < 4 / M::VEC; ++v) {
        typename M::vec_t y;
#pragma unroll
        for (int e = 0; e < M::VEC; ++e) y[e] = x[M::VEC * v + e];
        *reinterpret_cast<typename M::vec_t*>(row + M::VEC * v) = y;
      }
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t) row[t] = x[t];
    }
  }
}

// dS of the paired-range backward: per (batch, head) the causal 16 x 16
// tiles (query tile qt >= key tile j) back to back, tile (qt, j) at index
// qt (qt + 1) / 2 + j, each [query][key], so that a dQ-pass lane (query c)
// reads the four keys row(s, g) = 4g .. 4g + 3 it multiplies in MFMA steps
// s = 0..3 as one 16-byte vector.
__host__ __device__ inline int64_t ds16_tiles(int64_t nt) { return nt * (nt + 1) / 2; }

// Key pass. Block (bh, p), two waves, for the key tiles j = p and
// j' = nt - 1 - p of 16 keys (nt = T / 16 tiles, even), then for the pairs
// p + gridDim.y, ... when the grid is shortened to fit one round of resident
// blocks: key tile j is seen by the nt - p query tiles p .. nt - 1, key tile
// j' by p + 1, nt + 1 tile pairs in all. Wave 0 takes key tile j with query
// tiles p .. p + nt/2 - 1; wave 1 the rest of key tile j (query tiles
// p + nt/2 .. nt - 1), then all of key tile j'. Every wave thus carries nt/2
// or nt/2 + 1 tile pairs whatever p, and one two-way sum (key tile j's
// partial dK and dV, wave 0's first) remains.
// Each lane holds its key's K and V slices in registers; the query tiles'
// Q and dO rows pass through the wave's own LDS, the next one prefetched into
// registers. For each tile pair: S = Q K^T and dP = dO V^T, P recomputed from
// the forward's row max and sum, dS = P * (dP - rowsum(dO * O)) written to the
// workspace, dV^T += dO^T P and dK^T += Q^T dS.
// Aligned float32 path only: D = 64, T a multiple of 32, 16-byte access.
template <typename T>
__global__ void __launch_bounds__(128, 3) attn_bwd_kvp_kernel(AttnArgs a) {
  static_assert(sizeof(T) == 4, "float32 only");
  using M = A16<T>;
  typedef typename M::vec_t VT;
  typedef typename M::acc_t AT;
  constexpr int MT = 16, DP = 64, VEC = M::VEC;
  constexpr int LD = DP + VEC;                 // padded LDS row
  constexpr int TILE = MT * LD;
  constexpr int WAVE_LDS = 2 * TILE + 2 * MT;  // Q rows, dO rows, 2 statistics per row
  constexpr int NV = MT * DP / VEC / 64;       // 16-byte vectors per lane per tile and operand
  constexpr int RPV = 64 * VEC / DP;           // rows covered by one vector index
  constexpr int NF = 16 / VEC;                 // vectors of a lane's 16-element K / V slice
  constexpr int STASH = 2 * 4 * 4 * 64;        // wave 1's partial dK, dV of key tile j, register order
  __shared__ __attribute__((aligned(16))) T lds[2 * WAVE_LDS + STASH];

  const int bh = blockIdx.x;
  const int64_t b = bh / a.H, h = bh % a.H;
  const int Tn = (int)a.T, nt = Tn / MT, half = nt / 2;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4, c = lane & 15;
  const T* Q = (const T*)a.q + b * a.sq.b + h * a.sq.h;
  const T* K = (const T*)a.k + b * a.sk.b + h * a.sk.h;
  const T* Vv = (const T*)a.v + b * a.sv.b + h * a.sv.h;
  const T* G = (const T*)a.dO + b * a.sdo.b + h * a.sdo.h;
  const T* RM = (const T*)a.rowmax + (int64_t)bh * Tn;
  const T* RS = (const T*)a.rowsum + (int64_t)bh * Tn;
  const T* DR = (const T*)a.drow + (int64_t)bh * Tn;
  T* DS = (T*)a.ds + (int64_t)bh * ds16_tiles(nt) * (MT * MT);
  const T sl2 = (T)(a.scale * 1.4426950408889634);
  constexpr uint32_t S = sizeof(T);
  const Rsrc rQ = make_rsrc(Q, (uint64_t)Tn * a.sq.t * S), rG = make_rsrc(G, (uint64_t)Tn * a.sdo.t * S);
  const Rsrc rK = make_rsrc(K, (uint64_t)Tn * a.sk.t * S), rV = make_rsrc(Vv, (uint64_t)Tn * a.sv.t * S);
  const Rsrc rM = make_rsrc(RM, (uint64_t)Tn * S), rL = make_rsrc(RS, (uint64_t)Tn * S),
             rD = make_rsrc(DR, (uint64_t)Tn * S);
  const Rsrc rS = make_rsrc(DS, (uint64_t)ds16_tiles(nt) * MT * MT * S);

  T* Qs = lds + wave * WAVE_LDS;
  T* Gs = Qs + TILE;
  T* ST = Qs + 2 * TILE;  // [0, 16): max + log2(sum), [16, 32): rowsum(dO * O)
  T* stash = lds + 2 * WAVE_LDS;

  // this lane's share of a tile's loads: vector v is row RPV v + lrow, columns lcol ..
  const int lrow = lane / (DP / VEC), lcol = (lane % (DP / VEC)) * VEC;
  const uint32_t vq = (uint32_t)(lrow * a.sq.t + lcol) * S, vg = (uint32_t)(lrow * a.sdo.t + lcol) * S;
  const uint32_t vs = (uint32_t)c * S;
  VT rq[NV], rg[NV];
  T rm = T(0), rl = T(1), rd = T(0);
  auto fetch = [&](int qs) {
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      rq[v] = buf_load_v<VT>(rQ, vq, (uint32_t)((qs + RPV * v) * a.sq.t) * S);
      rg[v] = buf_load_v<VT>(rG, vg, (uint32_t)((qs + RPV * v) * a.sdo.t) * S);
    }
    rm = buf_load1(rM, vs, (uint32_t)qs * S);
    rl = buf_load1(rL, vs, (uint32_t)qs * S);
    rd = buf_load1(rD, vs, (uint32_t)qs * S);
  };
  auto put = [&]() {
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int r = RPV * v + lrow;
      *reinterpret_cast<VT*>(Qs + r * LD + lcol) = rq[v];
      *reinterpret_cast<VT*>(Gs + r * LD + lcol) = rg[v];
    }
    if (lane < MT) {
      ST[lane] = rm + log2(rl);
      ST[MT + lane] = rd;
    }
  };
  auto wave_sync = [] {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };

  // pairs p = blockIdx.y, + gridDim.y, ...: more than one when the grid would
  // otherwise run in several rounds of resident blocks
  for (int p = blockIdx.y; p < half; p += gridDim.y) {
    AT dk[4], dv[4];
    const int nseg = wave == 0 ? 1 : 2;
    for (int seg = 0; seg < nseg; ++seg) {
      const int j = seg == 0 ? p : nt - 1 - p;
      const int qa = seg == 1 ? j : (wave == 0 ? p : p + half);
      const int qb = wave == 0 ? p + half - 1 : nt - 1;
      const int k0 = j * MT;
      // this lane's key k0 + c: elements 16 g .. 16 g + 15 of its K and V rows
      VT kf[NF], vf[NF];
      const uint32_t kl = (uint32_t)((k0 + c) * a.sk.t + 16 * g) * S, vl = (uint32_t)((k0 + c) * a.sv.t + 16 * g) * S;
#pragma unroll
      for (int f = 0; f < NF; ++f) {
        kf[f] = buf_load_v<VT>(rK, kl, (uint32_t)(16 * f));
        vf[f] = buf_load_v<VT>(rV, vl, (uint32_t)(16 * f));
      }
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) dk[dt] = dv[dt] = AT(0);
      fetch(qa * MT);
      put();
      drain_vm();  // K and V slices in: the loop's waits then cover only its own prefetch
      wave_sync();
      for (int qt = qa; qt <= qb; ++qt) {
        const int qs = qt * MT;
        const bool more = qt < qb;
        if (more) fetch(qs + MT);
        // S(r, key) and dP(r, key): rows r = the tile's queries, column c = this lane's key
        AT s = AT(0), dp = AT(0);
#pragma unroll
        for (int f = 0; f < NF; ++f) {
          const VT x = *reinterpret_cast<const VT*>(Qs + c * LD + 16 * g + VEC * f);
          const VT y = *reinterpret_cast<const VT*>(Gs + c * LD + 16 * g + VEC * f);
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            s = M::mma(x[e], kf[f][e], s);
            dp = M::mma(y[e], vf[f][e], dp);
          }
        }
        auto probs = [&](auto maskc) {
          constexpr bool MASK = decltype(maskc)::value;  // the diagonal tile
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = M::row(i, g);
            T pr = ex2(__builtin_fmaf(s[i], sl2, -ST[r]));
            if constexpr (MASK) pr = c > r ? T(0) : pr;  // key above the query: masked
            s[i] = pr;
            dp[i] = pr * (dp[i] - ST[MT + r]);
          }
        };
        if (qt == j)
          probs(std::true_type());
        else
          probs(std::false_type());
        // dS tile (qt, j), [query][key]: queries row(i, g), this lane's key
        const uint32_t tb = (uint32_t)((qt * (qt + 1) / 2 + j) * (MT * MT)) * S;
#pragma unroll
        for (int i = 0; i < 4; ++i) buf_store1(dp[i], rS, (uint32_t)(M::row(i, g) * MT + c) * S, tb);
        // dV^T += dO^T P ; dK^T += Q^T dS: result tile t, row r is d = 4 r + t,
        // column = this lane's key, so a lane's A operands are dO and Q rows
        // row(i, g), d = 4c .. 4c + 3 (16-byte reads)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = M::row(i, g);
          VT gv[4 / VEC], qv[4 / VEC];
#pragma unroll
          for (int v = 0; v < 4 / VEC; ++v) {
            gv[v] = *reinterpret_cast<const VT*>(Gs + r * LD + 4 * c + VEC * v);
            qv[v] = *reinterpret_cast<const VT*>(Qs + r * LD + 4 * c + VEC * v);
          }
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            dv[t] = M::mma(gv[t / VEC][t % VEC], s[i], dv[t]);
            dk[t] = M::mma(qv[t / VEC][t % VEC], dp[i], dk[t]);
          }
        }
        wave_sync();
        if (more) put();
        wave_sync();
      }
      if (wave == 1) {
        if (seg == 0) {  // key tile j's later query tiles: handed to wave 0
#pragma unroll
          for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              stash[(dt * 4 + i) * 64 + lane] = dk[dt][i];
              stash[(16 + dt * 4 + i) * 64 + lane] = dv[dt][i];
            }
        } else {
          store_kv16<T>(a, b, h, k0, dk, dv, g, c);
        }
      }
    }
    __syncthreads();  // wave 1's partial of key tile j is in the stash
    if (wave == 0) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          dk[dt][i] += stash[(dt * 4 + i) * 64 + lane];
          dv[dt][i] += stash[(16 + dt * 4 + i) * 64 + lane];
        }
      store_kv16<T>(a, b, h, p * MT, dk, dv, g, c);
    }
    __syncthreads();  // the stash is read before the next pair writes it
  }
}

// dQ pass. Block (bh, bq) has eight waves for NDT pairs of query tiles, each
// query tile taken by 4 / NDT waves of NDT d-tiles (16 d each). With NDT = 4:
// wave w < 4 takes tile i = 4 bq + w, wave w + 4 its mirror i' = nt - 1 - i
// (i < nt / 2); with NDT = 2, waves w and w ^ 1 (w < 4) split tile
// i = 2 bq + w / 2 into d-tiles 0, 1 and 2, 3, and waves w + 4 its mirror.
// Tile i and its mirror see i + 1 and nt - i key tiles, nt + 1 in all, and
// waves w and w + 4 share a SIMD, so every SIMD carries the same work. NDT = 2
// is for short sequences, where four pairs per block leave the CUs unevenly
// loaded (B 16, H 12, T 256: 384 blocks on 256 CUs); it reads each dS tile
// twice. The block's waves walk the key tiles together, two per step (j = 2 it,
// 2 it + 1, up to the block's longest mirror tile), the step's K tiles staged
// in LDS once for all eight; a wave adds dS(q, j) K_j for the key tiles its
// query tile q sees. The next step's K and dS tiles are loaded at the top of a
// step and consumed at the next one. Output column c of the MFMA result tile t
// is d = 4 c + t, so that a lane's B operands (a K row, d = 4c + t for its
// d-tiles t, from LDS), its A operands (a dS row, stored [query][key]) and its
// dQ rows are vectors.
template <typename T, int NDT>
__global__ void __launch_bounds__(512, 2) attn_bwd_qp_kernel(AttnArgs a) {
  static_assert(sizeof(T) == 4, "float32 only");
  static_assert(NDT == 4 || NDT == 2, "d-tiles per wave");
  using M = A16<T>;
  typedef typename M::vec_t VT;
  typedef typename M::acc_t AT;
  typedef float HT __attribute__((ext_vector_type(NDT)));
  constexpr int MT = 16, DP = 64, VEC = M::VEC;
  constexpr int LD = DP + VEC;
  constexpr int KT = 2;                         // key tiles per step
  constexpr int STEP = KT * MT * LD;            // one step's K rows in LDS
  constexpr int NTH = 512;
  constexpr int KV = KT * MT * DP / VEC / NTH;  // K vectors per thread per step
  constexpr int SL = 4 / VEC;                   // vectors of a lane's dS row per tile
  constexpr int SPLIT = 4 / NDT;                // waves per query tile
  static_assert(KV * NTH * VEC == KT * MT * DP, "K rows: whole vectors per thread");
  __shared__ __attribute__((aligned(16))) T lds[2 * STEP];

  const int bh = blockIdx.x, bq = blockIdx.y;
  const int64_t b = bh / a.H, h = bh % a.H;
  const int Tn = (int)a.T, nt = Tn / MT, half = nt / 2;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4, c = lane & 15;
  const int i0 = NDT * bq + (wave & 3) / SPLIT;
  const int t0 = ((wave & 3) % SPLIT) * NDT;   // this wave's first d-tile
  const bool live = i0 < half;
  const int qt = wave < 4 ? i0 : nt - 1 - i0;  // this wave's query tile
  const int jend = nt - 1 - NDT * bq;          // the block's last key tile (the longest mirror tile)
  const int nstep = jend / KT + 1;
  constexpr uint32_t S = sizeof(T);
  const T* K = (const T*)a.k + b * a.sk.b + h * a.sk.h;
  const T* DS = (const T*)a.ds + (int64_t)bh * ds16_tiles(nt) * (MT * MT);
  const Rsrc rK = make_rsrc(K, (uint64_t)Tn * a.sk.t * S);
  const Rsrc rS = make_rsrc(DS, (uint64_t)ds16_tiles(nt) * MT * MT * S);

  int kro[KV], kco[KV];
#pragma unroll
  for (int v = 0; v < KV; ++v) {
    const int f = (int)threadIdx.x + NTH * v;
    kro[v] = f / (DP / VEC);
    kco[v] = (f % (DP / VEC)) * VEC;
  }
  const uint32_t svo = (uint32_t)(c * MT + 4 * g) * S;  // dS row c, keys 4g .. 4g + 3
  const int rq = live ? qt : jend;
  VT rk[KV], nx[KT][SL], xs[KT][SL];
  auto fetch = [&](int it) {
    const int j0 = KT * it;
#pragma unroll
    for (int v = 0; v < KV; ++v) {
      const int row = j0 * MT + kro[v];
      const int rowc = row < (jend + 1) * MT ? row : jend * MT + (kro[v] % MT);
      rk[v] = buf_load_v<VT>(rK, (uint32_t)kco[v] * S, (uint32_t)(rowc * a.sk.t) * S);
    }
#pragma unroll
    for (int u = 0; u < KT; ++u) {
      const int j = j0 + u;
      const uint32_t tb = (uint32_t)((rq * (rq + 1) / 2 + (j < rq ? j : rq)) * (MT * MT)) * S;
#pragma unroll
      for (int v = 0; v < SL; ++v) nx[u][v] = buf_load_v<VT>(rS, svo, tb + 16 * v);
    }
  };
  auto put = [&](T* Ks) {
#pragma unroll
    for (int v = 0; v < KV; ++v) *reinterpret_cast<VT*>(Ks + kro[v] * LD + kco[v]) = rk[v];
#pragma unroll
    for (int u = 0; u < KT; ++u)
#pragma unroll
      for (int v = 0; v < SL; ++v) xs[u][v] = nx[u][v];
  };
  AT dq[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t) dq[t] = AT(0);
  fetch(0);
  put(lds);
  __syncthreads();
  for (int it = 0; it < nstep; ++it) {
    const T* Ks = lds + (it & 1) * STEP;
    const bool more = it + 1 < nstep;
    if (more) fetch(it + 1);
#pragma unroll
    for (int u = 0; u < KT; ++u) {
      const int j = KT * it + u;
      if (live && j <= qt) {
        // dQ(r, d = 4c + t) += sum over the tile's keys of dS(r, key) K(key, d)
        HT kv[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
          kv[q] = *reinterpret_cast<const HT*>(Ks + (u * MT + M::row(q, g)) * LD + 4 * c + t0);
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int t = 0; t < NDT; ++t) dq[t] = M::mma(xs[u][q / VEC][q % VEC], kv[q][t], dq[t]);
      }
    }
    if (more) put(lds + ((it + 1) & 1) * STEP);
    __syncthreads();
  }
  if (live) {
    T* DQ = (T*)a.dq + b * a.sdq.b + h * a.sdq.h + 4 * c + t0;
    const T scale = (T)a.scale;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      T* row = DQ + (int64_t)(qt * MT + M::row(i, g)) * a.sdq.t;
      HT x;
#pragma unroll
      for (int t = 0; t < NDT; ++t) x[t] = dq[t][i] * scale;
      if (a.ovec) {
        *reinterpret_cast<HT*>(row) = x;
      } else {
#pragma unroll
        for (int t = 0; t < NDT; ++t) row[t] = x[t];
      }
    }
  }
}

template <typename T>
__device__ __forceinline__ T block_reduce_256(T x, T* red, bool is_max) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const T y = __shfl_xor(x, off, 64);
    x = is_max ? fmax(x, y) : x + y;
  }
  __syncthreads();  // red is free
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
  __syncthreads();
  return is_max ? fmax(fmax(red[0], red[1]), fmax(red[2], red[3])) : ((red[0] + red[1]) + red[2]) + red[3];
}

// Rows t of one batch element's S [H, T, T] (row r = h * T + t): P in place,
// row statistics to rowmax / rowsum at (b * H + h) * T + t (rowmax in base-2
// units, as the flash kernels keep it).
template <typename T>
__global__ void __launch_bounds__(256) attn_rows_softmax_kernel(T* __restrict__ S, T* __restrict__ rowmax,
                                                                 T* __restrict__ rowsum, int64_t Tn, int64_t row0,
                                                                 double scale) {
  __shared__ T red[4];
  const int64_t r = blockIdx.x;
  const int64_t t = r % Tn;
  T* sr = S + r * Tn;
  const T sc = (T)scale;
  T m = -INFINITY;
  for (int64_t j = threadIdx.x; j <= t; j += 256) m = fmax(m, sr[j] * sc);
  m = block_reduce_256(m, red, true);
  T l = T(0);
  for (int64_t j = threadIdx.x; j < Tn; j += 256) {
    const T p = j <= t ? exp(sr[j] * sc - m) : T(0);
    sr[j] = p;
    l += p;
  }
  l = block_reduce_256(l, red, false);
  const T linv = T(1) / l;
  for (int64_t j = threadIdx.x; j <= t; j += 256) sr[j] = sr[j] * linv;
  if (threadIdx.x == 0) {
    rowmax[row0 + r] = m * (T)1.4426950408889634;
    rowsum[row0 + r] = l;
  }
}

// P from S and the saved statistics, in place (entries above the diagonal 0).
template <typename T>
__global__ void __launch_bounds__(256) attn_rows_prob_kernel(T* __restrict__ S, const T* __restrict__ rowmax,
                                                              const T* __restrict__ rowsum, int64_t Tn, int64_t row0,
                                                              double scale) {
  const int64_t r = blockIdx.x;
  const int64_t t = r % Tn;
  T* sr = S + r * Tn;
  const T sl2 = (T)(scale * 1.4426950408889634);
  const T m = rowmax[row0 + r], linv = T(1) / rowsum[row0 + r];
  for (int64_t j = threadIdx.x; j < Tn; j += 256) sr[j] = j <= t ? ex2(sr[j] * sl2 - m) * linv : T(0);
}

// dS = P * (dP - rowsum(dP * P)) * scale, into dP.
template <typename T>
__global__ void __launch_bounds__(256) attn_rows_dsoft_kernel(const T* __restrict__ P, T* __restrict__ dP, int64_t Tn,
                                                               double scale) {
  __shared__ T red[4];
  const int64_t r = blockIdx.x;
  const T* pr = P + r * Tn;
  T* dr = dP + r * Tn;
  T s = T(0);
  for (int64_t j = threadIdx.x; j < Tn; j += 256) s += dr[j] * pr[j];
  s = block_reduce_256(s, red, false);
  const T sc = (T)scale;
  for (int64_t j = threadIdx.x; j < Tn; j += 256) dr[j] = pr[j] * (dr[j] - s) * sc;
}

// ----------------------------------------------------------------- host
static bool strides_vec(const Strides3& s, int64_t vec) { return s.b % vec == 0 && s.h % vec == 0 && s.t % vec == 0; }

template <typename T>
static int pick_dp(int64_t D) {
  constexpr int MT = AM<T>::MT;
  for (int dp : {16, 32, 64})
    if (dp >= MT && D <= dp) return dp;
  return -1;
}

#define DP_SWITCH_F(dp, KERNEL, T, grid, F)                                                  \
  switch (dp) {                                                                              \
    case 16: KERNEL<T, (sizeof(T) == 8 ? 16 : 32), F><<<grid, 256, 0, stream()>>>(a); break; \
    case 32: KERNEL<T, 32, F><<<grid, 256, 0, stream()>>>(a); break;                         \
    default: KERNEL<T, 64, F><<<grid, 256, 0, stream()>>>(a); break;                        \
  }
// FAST tile loads when 16-byte access is allowed and the head dimension fills the padded tile
#define DP_SWITCH(dp, KERNEL, T, grid)                                              \
  if (a.vec && a.D == (dp == 16 && sizeof(T) == 4 ? 32 : dp) && a.T % 128 == 0) { \
    DP_SWITCH_F(dp, KERNEL, T, grid, true)              \
  } else {                                               \
    DP_SWITCH_F(dp, KERNEL, T, grid, false)             \
  }

static int gemm_call(int dt, int akc, int bkc, int64_t M, int64_t N, int64_t K, const void* A, int64_t lda,
                     int64_t sA, const void* B, int64_t ldb, int64_t sB, void* C, int64_t ldc, int64_t sC,
                     int64_t batch) {
  return dtmi_gemm(dt, akc, bkc, M, N, K, A, lda, sA, B, ldb, sB, C, ldc, sC, batch, nullptr, 0, 0);
}

template <typename T>
static int attn_fwd_wide(AttnArgs& a) {
  const int dt = sizeof(T) == 4 ? DTMI_F32 : DTMI_F64;
  const int64_t B = a.B, H = a.H, Tn = a.T, D = a.D;
  void* S = nullptr;
  int rc = pool_alloc(&S, (size_t)H * Tn * Tn * sizeof(T));
  if (rc) return rc;
  for (int64_t b = 0; b < B && rc == 0; ++b) {
    const T* Q = (const T*)a.q + b * a.sq.b;
    const T* K = (const T*)a.k + b * a.sk.b;
    const T* V = (const T*)a.v + b * a.sv.b;
    T* O = (T*)a.out + b * a.so.b;
    // S[h] = Q[h] K[h]^T (the scale is applied in the row pass)
    rc = gemm_call(dt, 1, 1, Tn, Tn, D, Q, a.sq.t, a.sq.h, K, a.sk.t, a.sk.h, S, Tn, Tn * Tn, H);
    if (rc) break;
    {
      TimedLaunch tl(DTMI_FAM_ATTN_FWD, 0.0);
      attn_rows_softmax_kernel<T><<<(unsigned)(H * Tn), 256, 0, stream()>>>((T*)S, (T*)a.rowmax, (T*)a.rowsum, Tn,
                                                                             b * H * Tn, a.scale);
    }
    // O[h] = P[h] V[h]
    rc = gemm_call(dt, 1, 0, Tn, D, Tn, S, Tn, Tn * Tn, V, a.sv.t, a.sv.h, O, a.so.t, a.so.h, H);
  }
  hipError_t le = hipGetLastError();
  pool_free(S);
  if (rc) return rc;
  if (le != hipSuccess) return fail_hip(le, "attention (D > 64) kernels", __FILE__, __LINE__);
  return DTMI_OK;
}

template <typename T>
static int attn_bwd_wide(AttnArgs& a) {
  const int dt = sizeof(T) == 4 ? DTMI_F32 : DTMI_F64;
  const int64_t B = a.B, H = a.H, Tn = a.T, D = a.D;
  void* P = nullptr;
  void* dP = nullptr;
  int rc = pool_alloc(&P, (size_t)H * Tn * Tn * sizeof(T));
  if (rc) return rc;
  rc = pool_alloc(&dP, (size_t)H * Tn * Tn * sizeof(T));
  if (rc) {
    pool_free(P);
    return rc;
  }
  const int64_t TT = Tn * Tn;
  for (int64_t b = 0; b < B && rc == 0; ++b) {
    const T* Q = (const T*)a.q + b * a.sq.b;
    const T* K = (const T*)a.k + b * a.sk.b;
    const T* V = (const T*)a.v + b * a.sv.b;
    const T* G = (const T*)a.dO + b * a.sdo.b;
    T* dQ = (T*)a.dq + b * a.sdq.b;
    T* dK = (T*)a.dk + b * a.sdk.b;
    T* dV = (T*)a.dv + b * a.sdv.b;
    rc = gemm_call(dt, 1, 1, Tn, Tn, D, Q, a.sq.t, a.sq.h, K, a.sk.t, a.sk.h, P, Tn, TT, H);  // S
    if (rc) break;
    {
      TimedLaunch tl(DTMI_FAM_ATTN_BWD, 0.0);
      attn_rows_prob_kernel<T><<<(unsigned)(H * Tn), 256, 0, stream()>>>((T*)P, (const T*)a.rowmax,
                                                                          (const T*)a.rowsum, Tn, b * H * Tn, a.scale);
    }
    // dV = P^T dO: A(m = key, k = query) = P[query][key]
    rc = gemm_call(dt, 0, 0, Tn, D, Tn, P, Tn, TT, G, a.sdo.t, a.sdo.h, dV, a.sdv.t, a.sdv.h, H);
    if (rc) break;
    // dP = dO V^T
    rc = gemm_call(dt, 1, 1, Tn, Tn, D, G, a.sdo.t, a.sdo.h, V, a.sv.t, a.sv.h, dP, Tn, TT, H);
    if (rc) break;
    {
      TimedLaunch tl(DTMI_FAM_ATTN_BWD, 0.0);
      attn_rows_dsoft_kernel<T><<<(unsigned)(H * Tn), 256, 0, stream()>>>((const T*)P, (T*)dP, Tn, a.scale);
    }
    // dQ = dS K ; dK = dS^T Q
    rc = gemm_call(dt, 1, 0, Tn, D, Tn, dP, Tn, TT, K, a.sk.t, a.sk.h, dQ, a.sdq.t, a.sdq.h, H);
    if (rc) break;
    rc = gemm_call(dt, 0, 0, Tn, D, Tn, dP, Tn, TT, Q, a.sq.t, a.sq.h, dK, a.sdk.t, a.sdk.h, H);
  }
  hipError_t le = hipGetLastError();
  pool_free(P);
  pool_free(dP);
  if (rc) return rc;
  if (le != hipSuccess) return fail_hip(le, "attention backward (D > 64) kernels", __FILE__, __LINE__);
  return DTMI_OK;
}

// Forward on 16 x 16 tiles over paired ranges (float32 with 16-byte aligned
// Q, K and V, D = 64, T a multiple of 32): block (bh, p), one wave, query
// tile p and then its mirror nt - 1 - p, which see p + 1 and nt - p key
// tiles, nt + 1 in all, so every wave carries the same work (then the pairs
// p + gridDim.y, ... when the grid is shortened to one round of resident
// blocks). The wave's queries are the
// MFMA columns: S^T = K Q^T with K rows read from the wave's own LDS and the
// lane's Q slice (its query c, d = 16 g .. 16 g + 15, times scale * log2(e))
// in registers; P feeds O^T += V^T P^T from registers; the next key tile's K
// and V rows are prefetched into registers while the current one is computed.
// Lazy rescaling against a reference max as in attn_fwd_kernel.
__global__ void __launch_bounds__(64) attn_fwd_p16_kernel(AttnArgs a) {
  using M = A16<float>;
  typedef M::vec_t VT;
  typedef M::acc_t AT;
  constexpr int MT = 16, DP = 64, VEC = 4, LD = DP + VEC, TILE = MT * LD;
  constexpr int NV = MT * DP / VEC / 64;  // 16-byte vectors per lane per tile and operand
  constexpr int RPV = 64 * VEC / DP;      // rows per vector index
  constexpr int NF = 16 / VEC;            // vectors of a lane's 16-element Q slice
  __shared__ __attribute__((aligned(16))) float lds[2 * TILE];
  float* Ks = lds;
  float* Vs = lds + TILE;
  const int bh = blockIdx.x;
  const int64_t b = bh / a.H, h = bh % a.H;
  const int Tn = (int)a.T, nt = Tn / MT;
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, c = lane & 15;
  const float* Q = (const float*)a.q + b * a.sq.b + h * a.sq.h;
  const float* K = (const float*)a.k + b * a.sk.b + h * a.sk.h;
  const float* V = (const float*)a.v + b * a.sv.b + h * a.sv.h;
  float* O = (float*)a.out + b * a.so.b + h * a.so.h;
  const float sl2 = (float)(a.scale * 1.4426950408889634);
  constexpr uint32_t S = 4;
  const Rsrc rK = make_rsrc(K, (uint64_t)Tn * a.sk.t * S), rV = make_rsrc(V, (uint64_t)Tn * a.sv.t * S);
  const int lrow = lane / (DP / VEC), lcol = (lane % (DP / VEC)) * VEC;
  const uint32_t vk = (uint32_t)(lrow * a.sk.t + lcol) * S, vv = (uint32_t)(lrow * a.sv.t + lcol) * S;
  VT rk[NV], rv[NV];
  auto fetch = [&](int j) {
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      rk[v] = buf_load_v<VT>(rK, vk, (uint32_t)((j * MT + RPV * v) * a.sk.t) * S);
      rv[v] = buf_load_v<VT>(rV, vv, (uint32_t)((j * MT + RPV * v) * a.sv.t) * S);
    }
  };
  auto put = [&]() {
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int r = RPV * v + lrow;
      *reinterpret_cast<VT*>(Ks + r * LD + lcol) = rk[v];
      *reinterpret_cast<VT*>(Vs + r * LD + lcol) = rv[v];
    }
  };
  auto wave_sync = [] {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  auto gmax = [](float x) {
    x = fmaxf(x, __shfl_xor(x, 16, 64));
    return fmaxf(x, __shfl_xor(x, 32, 64));
  };
  // pairs p = blockIdx.y, + gridDim.y, ...: more than one when the grid would
  // otherwise run in several rounds of resident blocks
  for (int p = (int)blockIdx.y; p < nt / 2; p += (int)gridDim.y)
  for (int seg = 0; seg < 2; ++seg) {
    const int qt = seg == 0 ? p : nt - 1 - p;
    const int q0 = qt * MT;
    VT qf[NF];
    const float* qrow = Q + (int64_t)(q0 + c) * a.sq.t + 16 * g;
#pragma unroll
    for (int f = 0; f < NF; ++f) qf[f] = *reinterpret_cast<const VT*>(qrow + VEC * f) * sl2;
    AT o[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) o[t] = AT(0);
    float mref = -INFINITY, mtop = -INFINITY, l = 0.f;
    fetch(0);
    put();
    drain_vm();
    wave_sync();
    for (int j = 0; j <= qt; ++j) {
      const bool more = j < qt;
      if (more) fetch(j + 1);
      // S^T(key 4g + i, query c) in base-2 units
      AT s = AT(0);
#pragma unroll
      for (int f = 0; f < NF; ++f) {
        const VT x = *reinterpret_cast<const VT*>(Ks + c * LD + 16 * g + VEC * f);
#pragma unroll
        for (int e = 0; e < VEC; ++e) s = M::mma(x[e], qf[f][e], s);
      }
      if (j == qt) {  // the diagonal tile: keys after the query masked
#pragma unroll
        for (int i = 0; i < 4; ++i) s[i] = 4 * g + i > c ? -INFINITY : s[i];
      }
      float bmax = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
      mtop = fmaxf(mtop, bmax);
      if (__any(bmax > mref + kLazyLog2)) {
        const float mnew = fmaxf(mref, gmax(bmax));
        const float alpha = ex2(mref - mnew);  // mref = -inf on the first tile: 0
        l *= alpha;
#pragma unroll
        for (int t = 0; t < 4; ++t) o[t] *= alpha;
        mref = mnew;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        s[i] = ex2(s[i] - mref);
        l += s[i];
      }
      // O^T(d = 4 m + t, query c) += sum over the tile's keys of V(key, d) P(key, query)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const VT vr = *reinterpret_cast<const VT*>(Vs + (4 * g + i) * LD + 4 * c);
#pragma unroll
        for (int t = 0; t < 4; ++t) o[t] = M::mma(vr[t], s[i], o[t]);
      }
      wave_sync();
      if (more) put();
      wave_sync();
    }
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    mtop = gmax(mtop);
    const float inv = l > 0.f ? 1.f / l : 0.f;
    // lane (g, c) register i of tile t: d = 4 (4 g + i) + t of query c
    float* orow = O + (int64_t)(q0 + c) * a.so.t + 16 * g;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const VT x = {o[0][i] * inv, o[1][i] * inv, o[2][i] * inv, o[3][i] * inv};
      if (a.ovec) {
        *reinterpret_cast<VT*>(orow + 4 * i) = x;
      } else {  // O not 16-byte aligned: element stores, same values
#pragma unroll
        for (int t = 0; t < 4; ++t) orow[4 * i + t] = x[t];
      }
    }
    if (g == 0) {
      ((float*)a.rowmax)[(int64_t)bh * Tn + q0 + c] = mtop;
      ((float*)a.rowsum)[(int64_t)bh * Tn + q0 + c] = l * ex2(mref - mtop);
    }
    wave_sync();  // the last tile's rows are read before the next segment's put
  }
}

// Tile pairs per block of the paired-range forward and key pass. Their blocks
// all take the same time, so a grid of b blocks with s of them resident at
// once runs ceil(b / s) rounds; k pairs per block cost ceil(b_k / s) * k
// pair-times, b_k = bh * ceil(pairs / k). Take the cheapest k, the larger on a
// tie: each round starts with every block loading its first tiles at once and
// ends with all of them storing, which the rounds do not overlap (key pass at
// B 8, H 12, T 1024: two rounds of one pair 236 us, one round of two pairs
// 225 us). resident: blocks per CU (0 if unknown: one pair per block).
static unsigned pairs_per_block(int64_t bh, unsigned pairs, int resident) {
  const int64_t slots = (int64_t)resident * num_cus();
  if (slots <= 0) return 1;
  unsigned best = 1;
  int64_t best_cost = INT64_MAX;
  for (unsigned k = 1; k <= pairs && k <= 8; ++k) {
    const int64_t cost = cdiv(bh * cdiv((int64_t)pairs, (int64_t)k), slots) * k;
    if (cost <= best_cost) {
      best_cost = cost;
      best = k;
    }
  }
  return best;
}

template <typename F>
static int resident_blocks(F kernel, int threads) {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, threads, 0) != hipSuccess) n = 0;
  return n;
}

template <typename T>
static int attn_fwd_impl(AttnArgs& a) {
  constexpr int MT = AM<T>::MT;
  const int dp = pick_dp<T>(a.D);
  if (dp < 0) return attn_fwd_wide<T>(a);
  dim3 grid((unsigned)cdiv(a.T, 4 * MT), (unsigned)(a.B * a.H));
  // causal-exact FLOP: 2 GEMMs of 2*D*T(T+1)/2 per (b, h)
  TimedLaunch tl(DTMI_FAM_ATTN_FWD, 2.0 * 2.0 * a.B * a.H * a.D * (double)a.T * (a.T + 1) / 2.0);
  if constexpr (std::is_same<T, float>::value) {
    // D = 64, T a multiple of 32, 16-byte reads of Q, K and V: the
    // paired-range forward on 16 x 16 tiles (O aligned or not, same bits)
    if (a.vec && a.D == 64 && a.T % 32 == 0) {
      static const int resident = resident_blocks(attn_fwd_p16_kernel, 64);
      const unsigned pairs = (unsigned)(a.T / 32);
      const unsigned per = pairs_per_block(a.B * a.H, pairs, resident);
      attn_fwd_p16_kernel<<<dim3((unsigned)(a.B * a.H), (unsigned)cdiv(pairs, per)), 64, 0, stream()>>>(a);
      LAUNCH_CHECK("attn_fwd_p16_kernel");
      return DTMI_OK;
    }
  }
  DP_SWITCH(dp, attn_fwd_kernel, T, grid)
  LAUNCH_CHECK("attn_fwd_kernel");
  return DTMI_OK;
}

// Largest dS workspace (bytes) the backward takes from the pool; above it the
// dQ pass recomputes S, P and dP itself. 4 GiB by default; settable so that
// the recompute path can be exercised at any size.
static int64_t g_max_ds_bytes = (int64_t)4 << 30;

template <typename T>
static int attn_bwd_impl(AttnArgs& a, const void* drow_in) {
  constexpr int MT = AM<T>::MT;
  const int dp = pick_dp<T>(a.D);
  if (dp < 0) return attn_bwd_wide<T>(a);
  const int64_t rows = a.B * a.H * a.T;
  void* drow = nullptr;  // rowsum(dO * O): given, or computed below
  int rc = drow_in ? 0 : pool_alloc(&drow, (size_t)rows * sizeof(T));
  if (rc) return rc;
  a.drow = drow_in ? const_cast<void*>(drow_in) : drow;
  // float32, D = 64, T a multiple of 32, 16-byte access: the paired-range
  // kernels on 16 x 16 tiles, with dS in causal tiles (float64 keeps the
  // 64-key blocks: its key pass needs twice the registers)
  const bool pair16 = std::is_same<T, float>::value && a.vec && a.D == 64 && a.T % 32 == 0;
  // dS for the dQ pass: B*H*T*T elements (the causal tiles only on the
  // paired-range path), up to g_max_ds_bytes; beyond that the dQ pass
  // recomputes S, P and dP itself.
  a.ds = nullptr;
  const double ds_bytes = pair16 ? (double)a.B * a.H * (double)ds16_tiles(a.T / 16) * 256.0 * sizeof(T)
                                 : (double)a.B * a.H * a.T * a.T * sizeof(T);
  if (ds_bytes <= (double)g_max_ds_bytes) {
    rc = pool_alloc(&a.ds, (size_t)ds_bytes);
    if (rc) {
      pool_free(drow);
      return rc;
    }
  }
  {
    // causal-exact FLOP of the 5 backward GEMMs (S recompute, dV, dP, dQ, dK)
    TimedLaunch tl(DTMI_FAM_ATTN_BWD, 5.0 * 2.0 * a.B * a.H * a.D * (double)a.T * (a.T + 1) / 2.0);
    constexpr int VE = 16 / (int)sizeof(T);  // elements per 16-byte vector
    const bool drow64 = a.D == 64 && aligned(a.o, 16) && aligned(a.dO, 16) && strides_vec(a.so, VE) &&
                        strides_vec(a.sdo, VE);
    if (drow_in) {
    } else if (drow64) {
      attn_drow64_kernel<T><<<(unsigned)cdiv(rows, 32), 256, 0, stream()>>>(a);
    } else {
      attn_drow_kernel<T><<<(unsigned)cdiv(rows, 4), 256, 0, stream()>>>(a);
    }
    dim3 grid((unsigned)cdiv(a.T, 4 * MT), (unsigned)(a.B * a.H));
    if (pair16 && a.ds) {
      if constexpr (std::is_same<T, float>::value) {
        const unsigned pairs = (unsigned)(a.T / 32);
        static const int resident = resident_blocks(attn_bwd_kvp_kernel<float>, 128);
        const unsigned per = pairs_per_block(a.B * a.H, pairs, resident);
        attn_bwd_kvp_kernel<T><<<dim3((unsigned)(a.B * a.H), (unsigned)cdiv(pairs, per)), 128, 0, stream()>>>(a);
        // fewer than two four-pair blocks per CU: split the d-tiles instead
        if ((int64_t)a.B * a.H * cdiv(pairs, 4) < 2 * (int64_t)num_cus())
          attn_bwd_qp_kernel<T, 2><<<dim3((unsigned)(a.B * a.H), (unsigned)cdiv(pairs, 2)), 512, 0, stream()>>>(a);
        else
          attn_bwd_qp_kernel<T, 4><<<dim3((unsigned)(a.B * a.H), (unsigned)cdiv(pairs, 4)), 512, 0, stream()>>>(a);
      }
    } else {
      // 128-key (128-query) blocks; the dQ pass reads dS, or recomputes it
      // above the workspace bound
      if (a.ds) {
        DP_SWITCH(dp, attn_bwd_kv_kernel, T, grid)
      } else {  // the aligned key-block pass writes dS unconditionally
        DP_SWITCH_F(dp, attn_bwd_kv_kernel, T, grid, false)
      }
      if (a.ds) {
        DP_SWITCH(dp, attn_bwd_q_ds_kernel, T, grid)
      } else {
        DP_SWITCH(dp, attn_bwd_q_kernel, T, grid)
      }
    }
  }
  hipError_t le = hipGetLastError();
  pool_free(drow);
  if (a.ds) pool_free(a.ds);
  if (le != hipSuccess) return fail_hip(le, "attention backward kernels", __FILE__, __LINE__);
  return DTMI_OK;
}

static Strides3 s3(const int64_t* s) { return Strides3{s[0], s[1], s[2]}; }

}  // namespace dtmi

using namespace dtmi;

DTMI_EXPORT int dtmi_attn_fwd(int dtype, int64_t B, int64_t H, int64_t T, int64_t D, double scale, const void* q,
                              const int64_t* q_strides, const void* k, const int64_t* k_strides, const void* v,
                              const int64_t* v_strides, void* o, const int64_t* o_strides, void* rowmax,
                              void* rowsum) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_DTYPE_OK(dtype);
  DTMI_CHECK(B >= 0 && H >= 0 && T >= 0 && D > 0 && B * H < 65536, "dtmi_attn_fwd: bad shape (B*H must be < 65536)");
  if (B * H * T == 0) return DTMI_OK;
  DTMI_CHECK(q && k && v && o && rowmax && rowsum && q_strides && k_strides && v_strides && o_strides,
             "dtmi_attn_fwd: NULL pointer");
  AttnArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.out = o;
  a.rowmax = rowmax;
  a.rowsum = rowsum;
  a.sq = s3(q_strides);
  a.sk = s3(k_strides);
  a.sv = s3(v_strides);
  a.so = s3(o_strides);
  a.B = B;
  a.H = H;
  a.T = T;
  a.D = D;
  a.scale = scale;
  const int64_t vecn = dtype == DTMI_F32 ? 4 : 2;
  a.vec = (D % vecn == 0 && aligned(q, 16) && aligned(k, 16) && aligned(v, 16) && strides_vec(a.sq, vecn) &&
           strides_vec(a.sk, vecn) && strides_vec(a.sv, vecn))
              ? 1
              : 0;
  a.ovec = (D % vecn == 0 && aligned(o, 16) && strides_vec(a.so, vecn)) ? 1 : 0;
  if (dtype == DTMI_F32) return attn_fwd_impl<float>(a);
  return attn_fwd_impl<double>(a);
  DTMI_BODY_END
}

static int attn_bwd_entry(int dtype, int64_t B, int64_t H, int64_t T, int64_t D, double scale, const void* q,
                          const int64_t* q_strides, const void* k, const int64_t* k_strides, const void* v,
                          const int64_t* v_strides, const void* o, const int64_t* o_strides, const void* dO,
                          const int64_t* dO_strides, const void* rowmax, const void* rowsum, void* dq,
                          const int64_t* dq_strides, void* dk, const int64_t* dk_strides, void* dv,
                          const int64_t* dv_strides, const void* drow) {
  DTMI_REQUIRE_INIT();
  DTMI_DTYPE_OK(dtype);
  DTMI_CHECK(B >= 0 && H >= 0 && T >= 0 && D > 0 && B * H < 65536, "dtmi_attn_bwd: bad shape (B*H must be < 65536)");
  if (B * H * T == 0) return DTMI_OK;
  DTMI_CHECK(q && k && v && o && dO && rowmax && rowsum && dq && dk && dv, "dtmi_attn_bwd: NULL pointer");
  DTMI_CHECK(q_strides && k_strides && v_strides && o_strides && dO_strides && dq_strides && dk_strides && dv_strides,
             "dtmi_attn_bwd: NULL strides");
  AttnArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  a.dO = dO;
  a.dq = dq;
  a.dk = dk;
  a.dv = dv;
  a.rowmax = (void*)rowmax;
  a.rowsum = (void*)rowsum;
  a.sq = s3(q_strides);
  a.sk = s3(k_strides);
  a.sv = s3(v_strides);
  a.so = s3(o_strides);
  a.sdo = s3(dO_strides);
  a.sdq = s3(dq_strides);
  a.sdk = s3(dk_strides);
  a.sdv = s3(dv_strides);
  a.B = B;
  a.H = H;
  a.T = T;
  a.D = D;
  a.scale = scale;
  const int64_t vecn = dtype == DTMI_F32 ? 4 : 2;
  a.vec = (D % vecn == 0 && aligned(q, 16) && aligned(k, 16) && aligned(v, 16) && aligned(dO, 16) &&
           strides_vec(a.sq, vecn) && strides_vec(a.sk, vecn) && strides_vec(a.sv, vecn) &&
           strides_vec(a.sdo, vecn))
              ? 1
              : 0;
  a.ovec = (D % vecn == 0 && aligned(dq, 16) && aligned(dk, 16) && aligned(dv, 16) && strides_vec(a.sdq, vecn) &&
            strides_vec(a.sdk, vecn) && strides_vec(a.sdv, vecn))
               ? 1
               : 0;
  if (dtype == DTMI_F32) return attn_bwd_impl<float>(a, drow);
  return attn_bwd_impl<double>(a, drow);
}

DTMI_EXPORT int dtmi_attn_bwd(int dtype, int64_t B, int64_t H, int64_t T, int64_t D, double scale, const void* q,
                              const int64_t* q_strides, const void* k, const int64_t* k_strides, const void* v,
                              const int64_t* v_strides, const void* o, const int64_t* o_strides, const void* dO,
                              const int64_t* dO_strides, const void* rowmax, const void* rowsum, void* dq,
                              const int64_t* dq_strides, void* dk, const int64_t* dk_strides, void* dv,
                              const int64_t* dv_strides) {
  DTMI_BODY_BEGIN
  return attn_bwd_entry(dtype, B, H, T, D, scale, q, q_strides, k, k_strides, v, v_strides, o, o_strides, dO,
                        dO_strides, rowmax, rowsum, dq, dq_strides, dk, dk_strides, dv, dv_strides, nullptr);
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_attn_bwd_rowsum(int dtype, int64_t B, int64_t H, int64_t T, int64_t D, double scale,
                                     const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                                     const void* v, const int64_t* v_strides, const void* o, const int64_t* o_strides,
                                     const void* dO, const int64_t* dO_strides, const void* rowmax,
                                     const void* rowsum, const void* drow, void* dq, const int64_t* dq_strides,
                                     void* dk, const int64_t* dk_strides, void* dv, const int64_t* dv_strides) {
  DTMI_BODY_BEGIN
  DTMI_CHECK(drow != nullptr, "dtmi_attn_bwd_rowsum: NULL rowsum(dO * O)");
  return attn_bwd_entry(dtype, B, H, T, D, scale, q, q_strides, k, k_strides, v, v_strides, o, o_strides, dO,
                        dO_strides, rowmax, rowsum, dq, dq_strides, dk, dk_strides, dv, dv_strides, drow);
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_attn_set_ds_limit(int64_t bytes, int64_t* previous) {
  DTMI_BODY_BEGIN
  DTMI_CHECK(bytes >= 0, "dtmi_attn_set_ds_limit: negative limit");
  if (previous) *previous = g_max_ds_bytes;
  g_max_ds_bytes = bytes;
  return DTMI_OK;
  DTMI_BODY_END
}
