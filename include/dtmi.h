/*
 * libdtmi — C ABI of the MI355X (gfx950) backward / gradient / optimizer path
 * that stands in for dtrain's NumPy arithmetic.
 *
 * dtrain (siddhaantxsingh/DISTRIBUTED-TRAINING) is pure Python over NumPy and has
 * no FFI of its own; every function below replaces the NumPy expression(s) cited
 * next to it (paths relative to the dtrain source tree). The Python host package
 * `dtmi` binds these with ctypes and keeps dtrain's Python API on top.
 *
 * Conventions
 *   - Every function returns int status: 0 = ok, otherwise a DTMI_ERR_* code;
 *     dtmi_last_error() returns the (thread-local) message of the last failure.
 *   - dtype is DTMI_F32 or DTMI_F64. Pointers are device addresses (a buffer
 *     base plus a byte offset, so views and shards are plain pointers); sizes
 *     are int64_t element counts; arrays are row-major and contiguous unless a
 *     stride argument says otherwise.
 *   - Scalar hyper-parameters are passed as double, computed on the host the
 *     way dtrain computes them; F32 kernels round them to float first (NumPy 2
 *     treats Python floats as weak scalars of the array's dtype).
 *   - All work is enqueued on one library HIP stream, asynchronously. Errors of
 *     an asynchronous kernel surface at the next dtmi_sync / copy to host.
 *   - Reductions are deterministic: fixed grids, fixed combination order, no
 *     floating-point atomics. Same inputs give the same bits on every run.
 */
#ifndef DTMI_H
#define DTMI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DTMI_F32 0
#define DTMI_F64 1

#define DTMI_OK 0
#define DTMI_ERR_INVALID 1
#define DTMI_ERR_HIP 2
#define DTMI_ERR_OOM 3
#define DTMI_ERR_NOT_INITIALIZED 4
#define DTMI_ERR_INTERNAL 5

/* ------------------------------------------------------------------ runtime
 * Replaces: NumPy array allocation / np.zeros_like / .copy() behind
 * dtrain/autograd.py:43 (Tensor.data) and dtrain/autograd.py:181 (leaf .grad).
 */
const char* dtmi_last_error(void);
int dtmi_init(int device);                       /* select device, create the stream */
int dtmi_device_info(int* num_cus, size_t* hbm_bytes, char* name, int name_len);
int dtmi_malloc(void** ptr, size_t bytes);       /* pooled hipMalloc, 256-byte aligned */
int dtmi_free(void* ptr);                        /* back to the pool (stream ordered) */
int dtmi_empty_cache(void);                      /* release pooled blocks to HIP */
int dtmi_memory_stats(size_t* in_use, size_t* cached, size_t* peak);
int dtmi_memcpy_h2d(void* dst, const void* src, size_t bytes);   /* via pinned staging, async */
int dtmi_memcpy_d2h(void* dst, const void* src, size_t bytes);   /* synchronous */
int dtmi_memcpy_d2d(void* dst, const void* src, size_t bytes);
int dtmi_fill(int dtype, void* x, double value, int64_t n);      /* fill kernel (no hipMemset) */
int dtmi_zero_bytes(void* x, size_t bytes);
int dtmi_sync(void);

/* Timing: events on the library stream. */
int dtmi_event_create(void** ev);
int dtmi_event_record(void* ev);
int dtmi_event_elapsed_ms(void* start, void* stop, float* ms);   /* waits for stop */
int dtmi_event_destroy(void* ev);

/* Per-kernel-family timing of every launch while enabled (HIP events around
 * each launch on the library stream). Families are DTMI_FAM_*. */
#define DTMI_FAM_GEMM 0
#define DTMI_FAM_ATTN_FWD 1
#define DTMI_FAM_ATTN_BWD 2
#define DTMI_FAM_ADAMW 3
#define DTMI_FAM_BUCKET_AVG 4
#define DTMI_FAM_LN_BWD 5
#define DTMI_FAM_GELU_BWD 6
#define DTMI_FAM_XENT 7
#define DTMI_FAM_SUMSQ 8
#define DTMI_FAM_FLATTEN 9
#define DTMI_FAM_OTHER 10
#define DTMI_FAM_COUNT 11
int dtmi_timing_enable(int enable);              /* enabling clears the counters */
int dtmi_timing_read(int family, int64_t* launches, double* ms, double* work);

/* ---------------------------------------------------- optimizer / gradient path */

/* Fused AdamW over one flat buffer: one pass reads p, g, m, v and writes p, m, v.
 * Replaces dtrain/optim.py:21-33 (AdamW.step) for one array, including the
 * gradient pre-scale `p.grad * s` of dtrain/train.py:159 (gscale, 1.0 = none).
 * The operation order is exactly optim.py:28-33 and the library is built with
 * -ffp-contract=off, so F64 results are bit-identical to NumPy's.
 * c1 = 1 - b1 and c2 = 1 - b2 as Python computes them; b1t = 1 - b1**t and
 * b2t = 1 - b2**t with t already incremented (optim.py:22-24).
 * gscale_dev, when not NULL, points at a device double that replaces gscale
 * (the clip factor computed on the device by dtmi_clip_scale). */
int dtmi_adamw(int dtype, void* p, const void* g, void* m, void* v, int64_t n,
               double lr, double b1, double b2, double eps, double wd,
               double c1, double c2, double b1t, double b2t,
               double gscale, const double* gscale_dev);

/* Multi-tensor AdamW: the same update over `ntensors` (p, g, m, v, n) tuples in
 * one launch (dtrain/optim.py:25-33 iterates these in a Python loop). Tensors
 * with g == NULL are skipped (optim.py:26-27). Pointer arrays live on the host. */
int dtmi_adamw_multi(int dtype, int ntensors, void* const* p, const void* const* g,
                     void* const* m, void* const* v, const int64_t* n,
                     double lr, double b1, double b2, double eps, double wd,
                     double c1, double c2, double b1t, double b2t,
                     double gscale, const double* gscale_dev);

/* Bucket flatten: copy `nsrc` contiguous gradients back to back into dst.
 * Replaces the hook copy `b.buf[off:off+n] = p.grad.reshape(-1)` of
 * dtrain/ddp.py:73-81 (one launch per completed bucket instead of one copy per
 * parameter) and the ZeRO flatten of dtrain/zero.py:46-53. A NULL source
 * writes zeros (ddp.py:88-94, zero.py:49-50). */
int dtmi_bucket_flatten(int dtype, void* dst, const void* const* srcs, const int64_t* counts, int nsrc);

/* Fixed-order average of W replica rows of one bucket:
 *   out[i] = (((rep[0][i] + rep[1][i]) + rep[2][i]) + ...) * inv_w
 * rep[r] = replicas + r * replica_stride (elements). Replaces the direct
 * all-reduce order of dtrain/comm.py:374-391 (rank 0 first, then 1, 2, ...)
 * followed by `b.buf *= 1.0 / world` of dtrain/ddp.py:104-106 (and `g *= 1/W`
 * of dtrain/zero.py:55). Bit-exact to NumPy in F64 and F32.
 * If sumsq_partials is not NULL the kernel also writes one double per block
 * (the block's sum of out[i]^2, f64 accumulation) for dtmi_sumsq_finish; the
 * number of blocks is returned in *nblocks (call with sumsq_partials == NULL
 * and nblocks != NULL to query it first). */
int dtmi_bucket_average(int dtype, void* out, const void* replicas, int world, int64_t n,
                        int64_t replica_stride, double inv_w, double* sumsq_partials, int64_t* nblocks);

/* The same average with the rank order of dtrain's ring collectives: element i
 * lies in segment s (seg_start[s] <= i < seg_start[s + 1], seg_start[0] = 0,
 * the last segment ends at n) and is summed starting at rank seg_first[s]:
 * ((rep[f] + rep[f+1]) + ...) + rep[f-1] (indices mod world), then * inv_w.
 * Replaces the ring all-reduce of dtrain/comm.py:292-303 + 342-372 (chunk c
 * of a bucket, partition(n, W) of its buffer, summed starting at rank c;
 * dtrain/ddp.py's default algo) and the reduce-scatter of dtrain/zero.py:54
 * (shard r summed starting at rank r). The host computes where the chunks of
 * dtrain's bucket buffer (reverse parameter order) fall in this layout.
 * seg_start / seg_first are host arrays of nseg entries. sumsq_partials as
 * for dtmi_bucket_average (one launch, so at most 16 segments with it). */
int dtmi_bucket_average_ring(int dtype, void* out, const void* replicas, int world, int64_t n,
                             int64_t replica_stride, double inv_w, const int64_t* seg_start, const int* seg_first,
                             int nseg, double* sumsq_partials);

/* Deterministic sum of squares in f64 over `nt` tensors, two-stage (per-block
 * partials in a fixed grid, then one fixed-order pass). Replaces
 * sum(float(np.dot(g64, g64)) for each grad) of dtrain/train.py:155-156 and
 * dtrain/zero.py:56. The result is written to the device double *out_dev. */
int dtmi_sumsq(int dtype, const void* const* ptrs, const int64_t* counts, int nt, double* out_dev);

/* Final fixed-order pass over `count` per-block partials (from
 * dtmi_bucket_average), accumulated onto *out_dev if accumulate != 0. */
int dtmi_sumsq_finish(const double* partials, int64_t count, double* out_dev, int accumulate);

/* Clip factor on the device from a device sum of squares, exactly
 * dtrain/optim.py:49-52: n = sqrt(sq); 1.0 if n <= max_norm or n == 0 else
 * max_norm / (n + 1e-6). Writes *scale_dev (double) and *norm_dev (may be NULL). */
int dtmi_clip_scale(const double* sumsq_dev, double max_norm, double* scale_dev, double* norm_dev);

/* ------------------------------------------------------- generic tensor ops
 * Behind dtrain's Tensor operators (dtrain/autograd.py:76-148) and views.
 */

/* dst = src element by element over `shape` (ndim <= 8); element strides for
 * either side, NULL = contiguous. Materialises reshape/transpose of strided
 * views (dtrain/autograd.py:124-131 return NumPy views that later ops copy). */
int dtmi_copy_strided(int dtype, void* dst, const int64_t* dst_strides, const void* src,
                      const int64_t* src_strides, int ndim, const int64_t* shape);

/* out (contiguous, `shape`) = a OP b, OP: 0 add, 1 sub, 2 mul; element strides
 * of a and b over `shape` (0 on broadcast axes, NULL = contiguous).
 * dtrain/autograd.py:76-98 (NumPy broadcasting of a + b, a - b, a * b). */
#define DTMI_OP_ADD 0
#define DTMI_OP_SUB 1
#define DTMI_OP_MUL 2
int dtmi_binary(int dtype, int op, void* out, const void* a, const int64_t* a_strides, const void* b,
                const int64_t* b_strides, int ndim, const int64_t* shape);

/* out = x * alpha (alpha_dev, when not NULL, points at a device scalar of
 * dtype that replaces alpha). The loss scaling `loss * (1.0 / n_micro)` of
 * dtrain/train.py:138 and its backward (autograd.py:96-97). */
int dtmi_scale(int dtype, void* out, const void* x, int64_t n, double alpha, const void* alpha_dev);

/* tanh-GELU forward and backward, dtrain/autograd.py:133-144 (same formula and
 * operation order; tanh recomputed in the backward instead of saved). */
int dtmi_gelu_fwd(int dtype, void* y, const void* x, int64_t n);
int dtmi_gelu_bwd(int dtype, void* dx, const void* x, const void* dy, int64_t n);

/* ReLU forward / backward, dtrain/autograd.py:146-148. */
int dtmi_relu_fwd(int dtype, void* y, const void* x, int64_t n);
int dtmi_relu_bwd(int dtype, void* dx, const void* x, const void* dy, int64_t n);

/* Sum over the axes with reduce_mask[d] != 0 (kept axes in order into
 * contiguous out): Tensor.sum and _unbroadcast, dtrain/autograd.py:29-36, 111-117. */
int dtmi_reduce_sum(int dtype, void* out, const void* x, const int64_t* strides, int ndim,
                    const int64_t* shape, const int* reduce_mask);

/* Column sums of a row-major [rows, cols] matrix, deterministic two-stage
 * (64-row partials, then a fixed-order pass). The bias gradient
 * _unbroadcast(g, (N,)) of dtrain/autograd.py:29-36 for y = x @ w + b.
 * accumulate != 0 adds onto out. */
int dtmi_colsum(int dtype, void* out, const void* x, int64_t rows, int64_t cols, int accumulate);

/* ------------------------------------------------------------ LayerNorm
 * dtrain/autograd.py:207-223. Row-major [rows, cols]; one wave per row.
 * Forward saves the row mean and 1/sqrt(var + eps) for the backward (dtrain
 * keeps xh and rstd; xh is recomputed from x, mean and rstd).
 * Backward: dx = rstd * (gxh - mean(gxh) - xh * mean(gxh * xh)), gxh = dy * w;
 * dw = sum_rows(dy * xh); db = sum_rows(dy) (deterministic block partials).
 * accumulate: bit 0 adds dx onto the existing dx, bit 1 adds dw/db onto theirs. */
int dtmi_layernorm_fwd(int dtype, void* y, void* mean, void* rstd, const void* x, const void* w, const void* b,
                       int64_t rows, int64_t cols, double eps);
int dtmi_layernorm_bwd(int dtype, void* dx, void* dw, void* db, const void* dy, const void* x, const void* w,
                       const void* mean, const void* rstd, int64_t rows, int64_t cols, int accumulate);
/* dtmi_layernorm_bwd with dx = dx_addend + (the LayerNorm input gradient): the
 * backward engine's sum of a second gradient into one already pending for the
 * same tensor (dtrain/autograd.py:193, grads[k] + pg), done in the LayerNorm
 * pass instead of a separate add; the same bits. dx_addend is a separate
 * buffer (not dx); accumulate bit 0 must be clear, bit 1 as above. */
int dtmi_layernorm_bwd_add(int dtype, void* dx, void* dw, void* db, const void* dy, const void* x, const void* w,
                           const void* mean, const void* rstd, const void* dx_addend, int64_t rows, int64_t cols,
                           int accumulate);
/* dtmi_layernorm_bwd / _add with dy given as the nparts split-K partials of
 * the product that made it (dy_parts: nparts contiguous [rows, cols] arrays,
 * as dtmi_linear_bwd_dx_parts leaves them): dy = ((p0 + p1) + ...) in the
 * split-K sum's order, added as the rows are loaded, so the results equal
 * summing first and calling dtmi_layernorm_bwd(_add). dx_addend may be NULL;
 * it and the partials must not overlap dx. dtrain/autograd.py:216-222. */
int dtmi_layernorm_bwd_parts(int dtype, void* dx, void* dw, void* db, const void* dy_parts, int nparts, const void* x,
                             const void* w, const void* mean, const void* rstd, const void* dx_addend, int64_t rows,
                             int64_t cols, int accumulate);
/* dtmi_layernorm_bwd that allocates nothing. No counterpart in dtrain: it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Same
 * arguments, kernels and bits as dtmi_layernorm_bwd; its dgamma/dbeta column
 * partials go to a fixed 8 MiB device array per GPU (held until the process
 * ends) instead of the pool: 2 * min(512, ceil(rows / 8)) * cols * element
 * size must fit (float32 up to 2048 columns, float64 up to 1024, at any row
 * count), larger shapes return DTMI_ERR_INVALID before any launch. Calls that
 * overlap on one GPU (from other threads or streams) share the array and
 * race; calls on the library stream are ordered. Not timed by
 * dtmi_timing_enable (that creates events). */
int dtmi_layernorm_bwd_noalloc(int dtype, void* dx, void* dw, void* db, const void* dy, const void* x, const void* w,
                               const void* mean, const void* rstd, int64_t rows, int64_t cols, int accumulate);

/* --------------------------------------------------------- cross entropy
 * dtrain/autograd.py:250-266 over logits [rows, vocab] and int64 targets.
 * Forward writes the mean loss -(sum_r log p[r, t_r]) / rows to *loss and the
 * per-row max and sum of exp for the backward. Backward writes
 * dlogits = (exp(z - max) / sum - onehot(t)) * (g / rows) where g is *g_dev
 * (a device scalar of dtype) or g_host when g_dev is NULL. */
int dtmi_xent_fwd(int dtype, void* loss, void* rowmax, void* rowsum, const void* logits, const int64_t* targets,
                  int64_t rows, int64_t vocab);
int dtmi_xent_bwd(int dtype, void* dlogits, const void* logits, const void* rowmax, const void* rowsum,
                  const int64_t* targets, const void* g_dev, double g_host, int64_t rows, int64_t vocab);
/* Forward and gradient together, for a training step: the dtmi_xent_fwd outputs
 * plus dlogits for an upstream gradient of 1, i.e. (exp(z - max) / sum -
 * onehot(t)) / rows (dtrain/autograd.py:262-265 with g = 1). float32 rows of
 * up to 65536 logits are read once and dlogits written once; other shapes run
 * the two kernels above. dtmi_xent_grad_scale then multiplies dlogits (n
 * elements) in place by the device scalar *g_dev unless it is exactly 1. */
int dtmi_xent_fused(int dtype, void* loss, void* dlogits, void* rowmax, void* rowsum, const void* logits,
                    const int64_t* targets, int64_t rows, int64_t vocab);
int dtmi_xent_grad_scale(int dtype, void* dlogits, const void* g_dev, int64_t n);

/* Row-wise softmax backward dS = P * (dP - rowsum(dP * P)), the core of
 * dtrain/autograd.py:242 (without the 1/sqrt(d) factor). */
int dtmi_softmax_bwd(int dtype, void* ds, const void* p, const void* dp, int64_t rows, int64_t cols);

/* ------------------------------------------------------------- embedding
 * dtrain/autograd.py:199-204. Forward gathers weight rows by int64 index.
 * Backward reproduces np.add.at(zeros, idx, g) bit for bit: perm lists the
 * positions of idx stably sorted by value, segment s covers
 * perm[seg_start[s] .. seg_start[s+1]) and belongs to row seg_row[s]; each row
 * is the in-order sum of its positions' gradient rows. zero_fill != 0 clears
 * dweight first (rows nobody indexes stay zero). */
int dtmi_embedding_fwd(int dtype, void* out, const void* weight, const int64_t* idx, int64_t n_idx, int64_t vocab,
                       int64_t cols);
int dtmi_embedding_bwd(int dtype, void* dweight, const void* dout, const int32_t* perm, const int32_t* seg_start,
                       const int32_t* seg_row, int nseg, int64_t vocab, int64_t cols, int zero_fill);
/* The stable sort behind the backward, on the device (replaces the host-side
 * np.argsort(idx, kind="stable") of the index array; dtrain's np.add.at order,
 * dtrain/autograd.py:202). idx: n_idx int64 row ids in device memory; out, all
 * device memory: perm[n_idx], seg_start[n_idx + 1], seg_row[n_idx] and
 * nseg[1] (the segment count; seg_start[nseg] = n_idx). Deterministic. */
int dtmi_embedding_segments(const int64_t* idx, int64_t n_idx, int32_t* perm, int32_t* seg_start, int32_t* seg_row,
                            int32_t* nseg);
/* dtmi_embedding_bwd with the segment count read on the device (the output of
 * dtmi_embedding_segments over n_idx positions). */
int dtmi_embedding_bwd_segs(int dtype, void* dweight, const void* dout, const int32_t* perm, const int32_t* seg_start,
                            const int32_t* seg_row, const int32_t* nseg, int64_t n_idx, int64_t vocab, int64_t cols,
                            int zero_fill);

/* ------------------------------------------------------------ MFMA GEMM
 * C[b] = sum_k A(m,k) B(k,n) (+ bias[n]) (+ C[b] if accumulate), batched.
 * a_kcontig: A(m,k) = A[m*lda + k], else A[k*lda + m].
 * b_kcontig: B(k,n) = B[n*ldb + k], else B[k*ldb + n].
 * splits > 0 forces that many K splits (0 = chosen from the tile count).
 * dtrain/autograd.py:102-109: a @ b and its backward g @ b^T, a^T @ g
 * (batched over leading dimensions). */
int dtmi_gemm(int dtype, int a_kcontig, int b_kcontig, int64_t M, int64_t N, int64_t K, const void* A, int64_t lda,
              int64_t strideA, const void* B, int64_t ldb, int64_t strideB, void* C, int64_t ldc, int64_t strideC,
              int64_t batch, const void* bias, int accumulate, int splits);

/* Arithmetic of the float32 GEMMs (every dtmi_gemm / dtmi_linear_* call with
 * DTMI_F32; float64 is unaffected). No dtrain counterpart: dtrain's float32
 * matmul is NumPy's (dtrain/autograd.py:102-109).
 *  - DTMI_GEMM_MATH_F32 (default): float32 MFMA (v_mfma_f32_32x32x2_f32).
 *  - DTMI_GEMM_MATH_BF16X6: each float32 operand split exactly into three
 *    bf16 parts (a = a0 + a1 + a2, round-to-nearest-even at each step); the
 *    six partial products a_i b_j with i + j <= 2 run on the bf16 MFMA
 *    (v_mfma_f32_32x32x16_bf16, exact products, float32 accumulation). The
 *    dropped terms are below 2^-23 |a b| per product, about one float32
 *    rounding. Used for 16-byte aligned operands; others take the float32 MFMA.
 *    Inputs of magnitude above 3.38e38 (bf16 overflow) are out of its range. */
#define DTMI_GEMM_MATH_F32 0
#define DTMI_GEMM_MATH_BF16X6 1
int dtmi_set_gemm_math(int math);
int dtmi_get_gemm_math(int* math);

/* Linear layer y = x @ w + b (dtrain/nn.py:63-65) with X [M,K], W [K,N]:
 * forward Y = X W + b (bias fused in the epilogue, may be NULL);
 * dX = dY W^T (autograd.py:106); dW = X^T dY (autograd.py:107, the batch sum
 * of _unbroadcast folded into the reduction over M) and db = column sums of
 * dY (autograd.py:29-36 via the add node, may be NULL). */
int dtmi_linear_fwd(int dtype, void* Y, const void* X, const void* W, const void* b, int64_t M, int64_t K, int64_t N);
int dtmi_linear_bwd_dx(int dtype, void* dX, const void* dY, const void* W, int64_t M, int64_t K, int64_t N,
                       int accumulate);
int dtmi_linear_bwd_dw(int dtype, void* dW, void* db, const void* X, const void* dY, int64_t M, int64_t K, int64_t N,
                       int accumulate);

/* Linear with its neighbours fused into the GEMM epilogue, in the operation
 * order of the unfused graph:
 *  - residual != NULL: Y = residual + (X W + b), Block's `x + self.proj(...)`
 *    and `x + self.out(...)` (dtrain/nn.py:104-105, the add of autograd.py:76-84);
 *  - act != NULL: Y = X W + b is kept (the pre-activation) and act = gelu(Y)
 *    (dtrain/autograd.py:133-138 applied to Linear's output, nn.py:105).
 * The two are not combined in one call. */
int dtmi_linear_fwd_fused(int dtype, void* Y, void* act, const void* X, const void* W, const void* b,
                          const void* residual, int64_t M, int64_t K, int64_t N);
/* Y = residual + (X W + b) followed by the next LayerNorm of the block,
 * H = layer_norm(Y; ln_w, ln_b, eps) with its row mean and rstd [M]: Block's
 * `x + self.proj(...)` / `x + self.out(...)` (dtrain/nn.py:104-105) and the
 * ln2 / next block's ln1 / final ln that reads that x (nn.py:101, 105, 136;
 * autograd.py:207-214). When the product is split over K, the split sum, bias,
 * residual and LayerNorm run as one row pass (Y is still written: the
 * residual stream and the LayerNorm backward read it). The same bits as
 * dtmi_linear_fwd_fused followed by dtmi_layernorm_fwd. residual may be NULL. */
int dtmi_linear_fwd_ln(int dtype, void* Y, void* H, void* mean, void* rstd, const void* X, const void* W,
                       const void* b, const void* residual, const void* ln_w, const void* ln_b, double eps, int64_t M,
                       int64_t K, int64_t N);
/* dX = gelu'(pre) * (dY W^T): the Linear input gradient followed by the GELU
 * backward of autograd.py:139-143 (pre = the saved pre-activation [M, K]). */
int dtmi_linear_bwd_dx_gelu(int dtype, void* dX, const void* dY, const void* W, const void* pre, int64_t M, int64_t K,
                            int64_t N);
/* dX = dY W^T (autograd.py:106) for the projection that reads the attention
 * output X = o [M, K] (Block's self.proj(att), dtrain/nn.py:103-104), plus
 * the rowsum(dO * O) term of the attention backward (autograd.py:242: the
 * (dP * P).sum(-1) of the softmax backward) for each 64-wide head:
 * rowdot[(b H + h) T + t] = sum_d dX[m, 64 h + d] X[m, 64 h + d], m = b T + t,
 * H = K / 64 -- summed in the split-K pass that forms dX, else in a pass over
 * it; the same bits as dtmi_attn_bwd's own row pass, so dtmi_attn_bwd_rowsum
 * gives dtmi_attn_bwd's results. float32, X and dX contiguous and 16-byte
 * aligned, K % 64 == 0, M % T == 0. */
int dtmi_linear_bwd_dx_rowdot(int dtype, void* dX, const void* dY, const void* W, const void* X, void* rowdot,
                              int64_t M, int64_t K, int64_t N, int64_t T);
/* dtmi_linear_bwd_dx (dX = dY W^T, [M, K]) for a consumer that adds split-K
 * partials itself: when the product is split in s, 2 <= s <= max_parts, the s
 * raw partials are written to parts ([s][M][K]) and *nparts = s (a host
 * pointer); otherwise the finished dX is written to parts[0] and *nparts = 1.
 * parts holds max_parts * M * K elements. dtrain/autograd.py:106. */
int dtmi_linear_bwd_dx_parts(int dtype, void* parts, int max_parts, int* nparts, const void* dY, const void* W,
                             int64_t M, int64_t K, int64_t N);

/* ------------------------------------------------------- causal attention
 * dtrain/autograd.py:226-247: o = softmax(q k^T * scale + causal mask) v over
 * (B, H, T, D), the head dimension D contiguous (up to 64 in the fused MFMA
 * kernels; above 64 through materialised scores and batched GEMMs, one batch
 * element at a time); each *_strides argument points at three
 * element strides (b, h, t) of that operand, so q/k/v/o/dq/dk/dv may be views
 * into fused [B, T, 3, H, D] / [B, T, H, D] buffers. The forward writes o and
 * the per-row softmax statistics (contiguous [B, H, T]): rowmax = log2(e) *
 * max_j(q . k_j * scale) (base-2 units, the kernels use exp2) and rowsum =
 * sum_j exp(q . k_j * scale - max); the backward recomputes the probabilities
 * from them and writes dq, dk, dv (dtrain keeps the full probability tensor). */
int dtmi_attn_fwd(int dtype, int64_t B, int64_t H, int64_t T, int64_t D, double scale, const void* q,
                  const int64_t* q_strides, const void* k, const int64_t* k_strides, const void* v,
                  const int64_t* v_strides, void* o, const int64_t* o_strides, void* rowmax, void* rowsum);
int dtmi_attn_bwd(int dtype, int64_t B, int64_t H, int64_t T, int64_t D, double scale, const void* q,
                  const int64_t* q_strides, const void* k, const int64_t* k_strides, const void* v,
                  const int64_t* v_strides, const void* o, const int64_t* o_strides, const void* dO,
                  const int64_t* dO_strides, const void* rowmax, const void* rowsum, void* dq,
                  const int64_t* dq_strides, void* dk, const int64_t* dk_strides, void* dv,
                  const int64_t* dv_strides);
/* dtmi_attn_bwd with rowsum(dO * O) [B, H, T] already formed (by
 * dtmi_linear_bwd_dx_rowdot, in the pass that produced dO): the same results
 * without the backward's own row pass over o and dO. */
int dtmi_attn_bwd_rowsum(int dtype, int64_t B, int64_t H, int64_t T, int64_t D, double scale, const void* q,
                         const int64_t* q_strides, const void* k, const int64_t* k_strides, const void* v,
                         const int64_t* v_strides, const void* o, const int64_t* o_strides, const void* dO,
                         const int64_t* dO_strides, const void* rowmax, const void* rowsum, const void* drow,
                         void* dq, const int64_t* dq_strides, void* dk, const int64_t* dk_strides, void* dv,
                         const int64_t* dv_strides);
/* The backward's dQ pass reads the dS = P * (dP - rowsum(dO * O)) that its key
 * pass wrote to a pooled [B, H, T, T] workspace when that takes at most
 * `bytes` (default 4 GiB), and otherwise recomputes S, P and dP itself (the
 * same products as dtrain/autograd.py:239-246). Sets the bound (0: always
 * recompute) and returns the previous one in *previous (if not NULL). */
int dtmi_attn_set_ds_limit(int64_t bytes, int64_t* previous);

#ifdef __cplusplus
}
#endif

#endif /* DTMI_H */
