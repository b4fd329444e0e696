/*
 * oxihip.h — C-ABI of liboxihip, the MI355X (gfx950) device backend for the
 * oxitorch layer-kernel hot path.
 *
 * Every entry point is `extern "C"`, takes plain pointers, int64 sizes and
 * scalars, never throws, and returns an `oxi_status`. A non-zero status leaves
 * a user-facing message in a thread-local slot read by `oxi_hip_last_error()`.
 * This mirrors the reference error convention (Result inside, exceptions only
 * at the boundary, no panics across FFI: reference docs/error-handling.md:7-57)
 * and the variant set of `OxitorchError` (crates/oxi-core/src/lib.rs:186-211).
 *
 * All device pointers are HBM buffers obtained from `oxi_hip_alloc`. Float data
 * is fp32; ids/targets are int64. Launches are asynchronous on one per-process
 * HIP stream owned by the library; `oxi_hip_sync()` and the d2h copy wait for
 * it. Output buffers never alias inputs unless an entry point says so.
 *
 * Strided entry points take, for each operand, strides in ELEMENTS that are
 * already broadcast-expanded to the iteration `shape` (stride 0 = broadcast),
 * i.e. what reference crates/oxi-tensor/src/layout.rs:97-121
 * (`broadcast_strides`) produces. Rank is at most OXI_MAX_DIMS.
 */
#ifndef OXIHIP_H
#define OXIHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OXI_MAX_DIMS 8

/* Status codes: one per OxitorchError variant (crates/oxi-core/src/lib.rs:186-211).
 * The caller maps them to Python exceptions as crates/oxi-bindings/src/error.rs:22-32:
 * 1,2 -> ValueError; 3 -> NotImplementedError; 4,5 -> RuntimeError. */
typedef enum oxi_status {
  OXI_OK = 0,
  OXI_INVALID_ARGUMENT = 1,
  OXI_SHAPE_MISMATCH = 2,
  OXI_NOT_IMPLEMENTED = 3,
  OXI_OUT_OF_BOUNDS = 4,
  OXI_OTHER = 5
} oxi_status;

/* Unary registry, same names and order as F32_UNARY_OPS
 * (crates/oxi-tensor/src/ops.rs:125-202). OXI_UNARY_IDENTITY is a plain copy
 * (used to materialize views: Tensor::contiguous, lib.rs:230-240). */
enum {
  OXI_UNARY_NEG = 0, OXI_UNARY_ABS, OXI_UNARY_SQRT, OXI_UNARY_RSQRT, OXI_UNARY_EXP,
  OXI_UNARY_LOG, OXI_UNARY_LOG2, OXI_UNARY_LOG10, OXI_UNARY_SIN, OXI_UNARY_COS,
  OXI_UNARY_TANH, OXI_UNARY_RELU, OXI_UNARY_SIGMOID, OXI_UNARY_FLOOR, OXI_UNARY_CEIL,
  OXI_UNARY_ROUND, OXI_UNARY_SIGN, OXI_UNARY_SQUARE, OXI_UNARY_RECIPROCAL,
  OXI_UNARY_IDENTITY, OXI_UNARY_COUNT
};

/* Binary registry, F32_BINARY_OPS (ops.rs:55-91), then comparisons F32_CMP_OPS
 * (ops.rs:96-121) which write 1.0f / 0.0f as Tensor::cmp does (lib.rs:284-304). */
enum {
  OXI_BINARY_ADD = 0, OXI_BINARY_SUB, OXI_BINARY_MUL, OXI_BINARY_DIV, OXI_BINARY_POW,
  OXI_BINARY_MIN, OXI_BINARY_MAX,
  OXI_CMP_EQ, OXI_CMP_NE, OXI_CMP_LT, OXI_CMP_LE, OXI_CMP_GT, OXI_CMP_GE,
  OXI_BINARY_COUNT
};

/* Reduction kinds, same order as ReduceKind (ops.rs:222-238). */
enum {
  OXI_REDUCE_SUM = 0, OXI_REDUCE_MEAN, OXI_REDUCE_MAX, OXI_REDUCE_MIN,
  OXI_REDUCE_ARGMAX, OXI_REDUCE_ARGMIN, OXI_REDUCE_NORM
};

/* VJP mode of the norms. REF reproduces the reference graph, where
 * `.apply("rsqrt")` detaches the inverse std (python/oxitorch/nn/functional.py:232,239
 * + crates/oxi-bindings/src/lib.rs:682-710); EXACT is the full derivative. */
enum { OXI_NORM_VJP_REF = 0, OXI_NORM_VJP_EXACT = 1 };

/* GELU variants: TANH is the reference F.gelu (functional.py:194-199); ERF is
 * the exact 0.5x(1+erf(x/sqrt2)) that the reference lacks. */
enum { OXI_GELU_TANH = 0, OXI_GELU_ERF = 1 };

/* Activations a norm VJP can absorb (oxi_*_norm_act_bwd): the elementwise
 * ones (the two GELU values equal OXI_GELU_*) and softmax / log_softmax over
 * the last dim. OXI_ACT_NONE (the *_lead_sum entry points only) is the plain
 * norm VJP. */
enum {
  OXI_ACT_NONE = -1,
  OXI_ACT_GELU_TANH = 0, OXI_ACT_GELU_ERF = 1, OXI_ACT_SILU = 2,
  OXI_ACT_SOFTMAX = 3, OXI_ACT_LOG_SOFTMAX = 4
};

/* ------------------------------------------------------------------------ */
/* Runtime: device identity, memory, stream.                                */
/* Replaces the CPU-only device seam: Tensor::device (crates/oxi-tensor/src/lib.rs:192-196),
 * DeviceBackend/CpuBackend (crates/oxi-tensor/src/ops.rs:294-327) and
 * device_count (crates/oxi-bindings/src/lib.rs:781-785). */

/* Select and initialise `device`; creates the library stream. Idempotent. */
int oxi_hip_init(int device);
/* Number of visible HIP devices (0 when none; not an error). */
int oxi_hip_device_count(int* count);
/* Index of the initialised device, or -1. */
int oxi_hip_current_device(int* device);
/* The device the library is bound to, or, before the first device use, the
 * one it will bind: OXI_HIP_DEVICE (a device index) when set, else 0. Replaces
 * the index of the reference's Device (crates/oxi-core/src/lib.rs:139-146),
 * reported as "hip:N" by Tensor.device (bindings lib.rs:406-408). */
int oxi_hip_default_device(int* device);
/* Device storage: replaces the Arc<Vec<f32>> buffer (lib.rs:53-58). Blocks are
 * recycled by a stream-ordered caching allocator. `bytes == 0` yields NULL. */
int oxi_hip_alloc(size_t bytes, void** out);
int oxi_hip_free(void* ptr);
/* Return every cached (free) block to the driver. */
int oxi_hip_empty_cache(void);
/* Bytes currently handed out, and bytes held in the cache. */
int oxi_hip_memory_stats(size_t* in_use, size_t* cached);
/* Copies. h2d and d2d are stream-ordered; d2h waits for the stream. */
int oxi_hip_memcpy_h2d(void* dst, const void* src, size_t bytes);
int oxi_hip_memcpy_d2h(void* dst, const void* src, size_t bytes);
int oxi_hip_memcpy_d2d(void* dst, const void* src, size_t bytes);
/* Transfers that do not stall the library stream (the step before the hot
 * path: ids, targets and loader batches reaching the device). Replaces the
 * CPU-only movement of Tensor::to / .cpu() and the loader's host batches
 * (plan.md:266-268; crates/oxi-data/src/batch.rs:411-423). */
/* Page-locked host memory; oxi_hip_host_free waits for queued copies first. */
int oxi_hip_host_alloc(size_t bytes, void** out);
int oxi_hip_host_free(void* ptr);
/* Upload from any host memory: the bytes are copied into a pinned staging
 * ring and the DMA is queued on the library stream; returns as soon as `src`
 * may be reused, without waiting for the device. */
int oxi_hip_upload(void* dst, const void* src, size_t bytes);
/* Queue a DMA from page-locked memory (oxi_hip_host_alloc) on the library
 * stream without waiting; `pinned_src` must stay unchanged until the stream
 * has passed the copy (oxi_hip_sync, or an event). */
int oxi_hip_memcpy_h2d_async(void* dst, const void* pinned_src, size_t bytes);
/* Download through the pinned ring, chunked and double-buffered; waits for
 * the queued work and the copy. */
int oxi_hip_download(void* dst, const void* src, size_t bytes);
/* Wait for all queued work; reports a pending device-side guard (e.g. an id
 * that escaped host validation) as OXI_OUT_OF_BOUNDS. */
int oxi_hip_sync(void);
/* Thread-local message of the last failing call on this thread ("" if none). */
const char* oxi_hip_last_error(void);
/* The library stream (a hipStream_t), for callers that time or order work. */
int oxi_hip_stream(void** stream);
/* Events on the library stream, for timing kernels (created without the
 * system-scope fence, which would flush the caches at every record). */
int oxi_hip_event_create(void** event);
int oxi_hip_event_record(void* event);
int oxi_hip_event_elapsed_ms(void* start, void* stop, float* ms);
int oxi_hip_event_destroy(void* event);
/* Properties of the initialised device, for reports (memory clock and bus
 * width as the runtime gives them; the HBM peak they imply is the caller's
 * to derive). */
typedef struct oxi_device_props {
  int32_t compute_units;
  int32_t memory_clock_khz;
  int32_t memory_bus_bits;
  int32_t l2_bytes;
  int64_t hbm_bytes;
  char arch[64];
} oxi_device_props;
int oxi_hip_device_props(oxi_device_props* out);
/* Test hook: make the next `n`-th allocation fail (0 disables). */
int oxi_hip_debug_fail_alloc_after(int n);

/* ------------------------------------------------------------------------ */
/* Elementwise registry on strided/broadcast operands.                      */
/* Strides are in elements, one per dim of `shape` (0 for a broadcast dim);  */
/* with ndim == 0 (a single element) `shape` and the stride arrays may be    */
/* NULL.                                                                     */

/* y = fill value (n contiguous floats). Used for Tensor::zeros/full
 * (lib.rs:67-158) and the scalar-operand promotion of const_full
 * (crates/oxi-bindings/src/lib.rs:86-89). Kernel fill, safe under graph capture. */
int oxi_fill(float* y, int64_t n, float value);

/* y[i] = op(x[i]) over `shape`. Replaces Tensor::unary / unary_op
 * (crates/oxi-tensor/src/lib.rs:306-325,353-357) and iterate::map_n
 * (crates/oxi-tensor/src/iterate.rs:21-75). */
int oxi_unary(int op, const float* x, const int64_t* x_strides,
              float* y, const int64_t* y_strides,
              const int64_t* shape, int ndim);

/* y[i] = a[i] op b[i] with broadcast strides. Replaces Tensor::binary /
 * binary_op / cmp_op (crates/oxi-tensor/src/lib.rs:263-304,332-347). */
int oxi_binary(int op, const float* a, const int64_t* a_strides,
               const float* b, const int64_t* b_strides,
               float* y, const int64_t* y_strides,
               const int64_t* shape, int ndim);

/* ------------------------------------------------------------------------ */
/* Fused activations (strided, one graph node each).                         */

/* F.gelu (python/oxitorch/nn/functional.py:194-199), `approximate` = OXI_GELU_*. */
int oxi_gelu_fwd(const float* x, const int64_t* x_strides,
                 float* y, const int64_t* y_strides,
                 const int64_t* shape, int ndim, int approximate);
/* dx = g * gelu'(x). For OXI_GELU_TANH the arithmetic follows the composed VJP
 * of the reference graph (mul/add/tanh VJPs, crates/oxi-autograd/src/ops.rs:62-73,218-230). */
int oxi_gelu_bwd(const float* x, const int64_t* x_strides,
                 const float* g, const int64_t* g_strides,
                 float* dx, const int64_t* dx_strides,
                 const int64_t* shape, int ndim, int approximate);
/* F.silu = x * sigmoid(x) (functional.py:202-204). */
int oxi_silu_fwd(const float* x, const int64_t* x_strides,
                 float* y, const int64_t* y_strides,
                 const int64_t* shape, int ndim);
/* dx = g*s + (g*x)*(s*(1-s)), the mul VJP (ops.rs:62-73) plus the sigmoid VJP (ops.rs:236-247). */
int oxi_silu_bwd(const float* x, const int64_t* x_strides,
                 const float* g, const int64_t* g_strides,
                 float* dx, const int64_t* dx_strides,
                 const int64_t* shape, int ndim);

/* ------------------------------------------------------------------------ */
/* Norms over the last dim of a contiguous (rows, cols) buffer.              */

/* F.rms_norm (functional.py:236-240): y = (x*inv)*w, inv = 1/sqrt(mean(x*x)+eps).
 * Writes the per-row `rstd` (= inv) for the backward. */
int oxi_rms_norm_fwd(const float* x, const float* w, float* y, float* rstd,
                     int64_t rows, int64_t cols, float eps);
/* RMS VJP. mode REF: dx = (g*w)*inv; EXACT: dx = inv*(g*w - xhat*mean(g*w*xhat)).
 * dw = sum over rows of g*(x*inv) (unbroadcast, crates/oxi-autograd/src/graph.rs:274-313).
 * dx or dw may be NULL to skip. Deterministic (no float atomics). */
int oxi_rms_norm_bwd(const float* x, const float* w, const float* rstd, const float* g,
                     float* dx, float* dw, int64_t rows, int64_t cols, int mode);
/* F.layer_norm (functional.py:227-233): y = ((x-mu)*inv)*w + b. w/b may be NULL
 * (no affine). Writes per-row mean and rstd. */
int oxi_layer_norm_fwd(const float* x, const float* w, const float* b, float* y,
                       float* mean, float* rstd, int64_t rows, int64_t cols, float eps);
/* LN VJP. mode REF: dx = gc - mean_row(gc), gc = (g*w)*inv; EXACT: the full
 * derivative. dw = sum_rows g*((x-mu)*inv), db = sum_rows g. dx/dw/db may be NULL. */
int oxi_layer_norm_bwd(const float* x, const float* w, const float* mean, const float* rstd,
                       const float* g, float* dx, float* dw, float* db,
                       int64_t rows, int64_t cols, int mode);
/* Fixed device scratch of oxi_layer_norm_bwd_noalloc, per device, held until
 * the process ends. */
#define OXI_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)
/* oxi_layer_norm_bwd without any allocation. This entry point has no
 * counterpart in the reference; it is for callers that cannot allocate device
 * memory: code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc. Same arguments and results as oxi_layer_norm_bwd (the
 * same kernels and launch shapes, so the outputs are bit-identical); the
 * column partials of dw/db (2 x blocks x cols floats, at most 2 x CUs x cols
 * for rows wider than 768 floats) live in a fixed OXI_NOALLOC_SCRATCH_BYTES
 * array in device memory instead of a workspace: on a 256-CU MI355X that
 * covers rows of up to 8192 floats. Larger sizes are refused with
 * OXI_INVALID_ARGUMENT before anything
 * is launched, and so is a call before oxi_hip_init (initialisation
 * allocates). Every call on one device shares the array and leaves it
 * holding its partials; nothing in it needs to start at zero. Calls from
 * several host threads are serialised, but calls that overlap on the device
 * (e.g. a captured graph replayed on another stream while a call runs on the
 * library stream) race on the array. */
int oxi_layer_norm_bwd_noalloc(const float* x, const float* w, const float* mean, const float* rstd,
                               const float* g, float* dx, float* dw, float* db,
                               int64_t rows, int64_t cols, int mode);
/* The VJPs of act(norm(x)) in one pass, for a graph where the norm's output y
 * feeds only the activation `act` (OXI_ACT_*). They replace the activation's
 * VJP followed by the norm's, which the reference runs as two graph nodes in
 * reverse topological order (crates/oxi-autograd/src/graph.rs:398-436: the
 * activation node's VJP accumulates y's gradient, the norm node's VJP reads
 * it). `g` is the gradient of act(y). y is recomputed from x and the saved
 * statistics with the forward's arithmetic; dy is the value oxi_gelu_bwd /
 * oxi_silu_bwd (g * act'(y)) or oxi_softmax_bwd / oxi_log_softmax_bwd (on the
 * softmax of y, recomputed as oxi_*softmax_fwd forms it) write, and is stored
 * to `dy` unless NULL (it is y's gradient, which the graph keeps); dx/dw/db
 * are what the matching oxi_*_norm_bwd computes from dy, bit for bit. Each row
 * then crosses HBM four times (read x and g, write dy and dx) instead of six.
 * Returns OXI_NOT_IMPLEMENTED and writes nothing when a row does not
 * vectorize (cols % 4 != 0, cols > 8192, or a pointer not 16-byte aligned),
 * or, for the softmax kinds, when cols > 2048: the caller then runs the two
 * VJPs. */
int oxi_rms_norm_act_bwd(const float* x, const float* w, const float* rstd, const float* g, int act,
                         float* dy, float* dx, float* dw, int64_t rows, int64_t cols, int mode);
int oxi_layer_norm_act_bwd(const float* x, const float* w, const float* b, const float* mean,
                           const float* rstd, const float* g, int act, float* dy, float* dx,
                           float* dw, float* db, int64_t rows, int64_t cols, int mode);

/* The norm VJP (act = OXI_ACT_NONE) or the norm + activation VJP above, over
 * rows that form a (lead, T) grid (rows = lead * T), that also writes
 * dx_sum (T, cols): dx_sum[t] = dx[0*T + t] + dx[1*T + t] + ... in batch
 * order, summed from 0.0f in f32, bit-identical to oxi_reduce(OXI_REDUCE_SUM)
 * over the leading dim of dx. That is the gradient of a (1, T, cols) operand
 * broadcast over the leading dim and added to the norm input (a positional
 * table): the reference forms it after the add's VJP, with unbroadcast
 * (crates/oxi-autograd/src/graph.rs:274-313, a strided serial column sum,
 * crates/oxi-tensor/src/lib.rs:549-558), a pass over dx of its own. dy, dx, dw
 * (and db) are what oxi_*_norm_bwd / oxi_*_norm_act_bwd write, bit for bit;
 * dx and dx_sum must not be NULL. OXI_NOT_IMPLEMENTED (nothing written) unless
 * the rows vectorize as oxi_*_norm_act_bwd requires, cols <= 1024 (one wave
 * per row) and lead is a multiple of 4: the caller then runs the VJP and the
 * reduction. dw and db
 * are the column sums the other entry points form, added in another row
 * order (deterministic, not bit-identical to them). This pass has no
 * counterpart in the reference. */
int oxi_rms_norm_bwd_lead_sum(const float* x, const float* w, const float* rstd, const float* g, int act,
                              float* dy, float* dx, float* dw, float* dx_sum, int64_t lead, int64_t rows,
                              int64_t cols, int mode);
int oxi_layer_norm_bwd_lead_sum(const float* x, const float* w, const float* b, const float* mean,
                                const float* rstd, const float* g, int act, float* dy, float* dx, float* dw,
                                float* db, float* dx_sum, int64_t lead, int64_t rows, int64_t cols, int mode);

/* ------------------------------------------------------------------------ */
/* Softmax family over the middle dim of a contiguous (outer, len, inner)    */
/* buffer (inner == 1 is the last-dim case).                                 */

/* F.softmax (functional.py:211-215). */
int oxi_softmax_fwd(const float* x, float* y, int64_t outer, int64_t len, int64_t inner);
/* dx = y*(g - sum(g*y)). */
int oxi_softmax_bwd(const float* y, const float* g, float* dx,
                    int64_t outer, int64_t len, int64_t inner);
/* F.log_softmax (functional.py:218-222). */
int oxi_log_softmax_fwd(const float* x, float* y, int64_t outer, int64_t len, int64_t inner);
/* dx = g - exp(y)*sum(g). */
int oxi_log_softmax_bwd(const float* y, const float* g, float* dx,
                        int64_t outer, int64_t len, int64_t inner);
/* F.cross_entropy, mean reduction (functional.py:277-293), fused: writes the
 * scalar loss (1 float on device) and the per-row log-sum-exp `lse` (n floats).
 * `targets` are int64 class ids already resolved to [0, c). As the reference's
 * sum(onehot * log_softmax(x)) does, a row whose non-target log-probability is
 * -inf (a -inf logit, or x - max overflowing) makes the loss NaN (0 * -inf);
 * lse and the gradient stay finite there. n == 0 writes a loss of -0.0 (the
 * reference's mean of no rows is 0, bindings lib.rs:126-143, negated). */
int oxi_cross_entropy_fwd(const float* logits, const int64_t* targets,
                          float* loss, float* lse, int64_t n, int64_t c);
/* dlogits = (softmax(logits) - onehot(targets)) * gloss[0] / n. `gloss` is a
 * device pointer to the upstream scalar gradient. */
int oxi_cross_entropy_bwd(const float* logits, const int64_t* targets, const float* lse,
                          const float* gloss, float* dlogits, int64_t n, int64_t c);
/* oxi_cross_entropy_fwd and oxi_cross_entropy_bwd for gloss = 1 in one pass
 * over the logits (no single reference counterpart: the composition of
 * functional.py:277-293 and its VJPs, for a backward seeded with 1, as
 * loss.backward() seeds it). Writes loss and lse as oxi_cross_entropy_fwd
 * does, bit for bit, and dlogits as the composed log_softmax VJP forms them:
 * (1/n)(1/s) exp(x - max) with s the row's sum of exp(x - max), less 1/n at
 * the target (oxi_cross_entropy_bwd, which has only lse, writes
 * (exp(x - lse) - onehot)/n; the two agree to within the reference path's
 * tolerance, not bit for bit). Needs c % 4 == 0 and 16-byte aligned logits and dlogits; other shapes
 * return OXI_NOT_IMPLEMENTED before any launch (take the two calls then). */
int oxi_cross_entropy_fwd_grad(const float* logits, const int64_t* targets, float* loss, float* lse,
                               float* dlogits, int64_t n, int64_t c);

/* ------------------------------------------------------------------------ */
/* Gather / scatter-add.                                                     */

/* out[o, k, i] = src[o, idx[k], i] for a contiguous (outer, len, inner) source.
 * `idx` (n int64 on device) may hold negatives in [-len, len), which wrap.
 * Replaces Tensor::index_select (crates/oxi-tensor/src/lib.rs:665-703); ids are
 * also validated on the host, this kernel only guards (see oxi_hip_sync). */
int oxi_index_select(const float* src, int64_t outer, int64_t len, int64_t inner,
                     const int64_t* idx, int64_t n, float* out);
/* Dense VJP of index_select: grad_src[o, v, i] = sum over k with idx[k]==v of
 * g[o, k, i], accumulated in position order k per id (a stable counting sort
 * by id plus a segmented reduction; no atomics on floats). Every element of
 * `grad_src` (outer*len*inner) is written. Replaces scatter_index_select
 * (crates/oxi-autograd/src/ops.rs:741-769). */
int oxi_index_select_bwd(const float* g, int64_t outer, int64_t len, int64_t inner,
                         const int64_t* idx, int64_t n, float* grad_src);
/* The same VJP in two halves, so the id-dependent half leaves the backward:
 * _plan sorts the ids (a stable sort by id with each id's presence flag) on
 * the library's second stream, after everything already queued on the library
 * stream, as soon as the ids are known (at forward time); _apply makes the
 * library stream wait for the plan and runs the segment sums of g for any
 * (outer, inner) of the same ids. A plan may be applied more than once.
 * _plan_free releases it (after the library stream has passed its sort).
 * Together they compute exactly what oxi_index_select_bwd computes. The
 * plan/apply split has no counterpart in the reference (its VJP is one call,
 * scatter_index_select, crates/oxi-autograd/src/ops.rs:741-769). */
int oxi_index_select_bwd_plan(const int64_t* idx, int64_t n, int64_t len, void** plan);
int oxi_index_select_bwd_apply(const void* plan, const float* g, int64_t outer, int64_t inner,
                               float* grad_src);
int oxi_index_select_bwd_plan_free(void* plan);

/* One batch of a column-tensor loader: dst[k, i] = src[idx[k], i] for every
 * column (src contiguous (len, inner), dst (n, inner)), all columns in one
 * launch (more than 8 columns take one launch per 8). Replaces
 * gather_columns (crates/oxi-data/src/batch.rs:406-423: index_select(0,
 * indices) per column). Ids in [-len, len) wrap; the caller validates them,
 * this kernel only guards (see oxi_hip_sync). */
typedef struct oxi_batch_column {
  const float* src;
  float* dst;
  int64_t inner;
} oxi_batch_column;
int oxi_batch_gather(const oxi_batch_column* cols, int ncols, int64_t len, const int64_t* idx, int64_t n);
/* F.embedding (functional.py:245-247) = index_select on dim 0 of W (V, D). */
int oxi_embedding_fwd(const float* W, const int64_t* ids, int64_t n,
                      int64_t V, int64_t D, float* out);
/* dW (V, D) = dense duplicate-accumulating VJP of F.embedding. */
int oxi_embedding_bwd(const float* g, const int64_t* ids, int64_t n,
                      int64_t V, int64_t D, float* dW);

/* Row scatter, last write wins: out (rows, inner) = base with row idx[p]
 * replaced by values row p, for p in order, so a row written twice keeps the
 * later values. `idx` (n int64 on device) may hold negatives in [-rows, rows),
 * which wrap; ids are validated on the host, the kernels only guard. base,
 * values and out are contiguous; out must not alias them. Replaces
 * Tensor::scatter_dim0 (crates/oxi-tensor/src/lib.rs:895-932). */
int oxi_scatter_rows(const float* base, int64_t rows, int64_t inner,
                     const int64_t* idx, int64_t n, const float* values, float* out);
/* VJP of the row scatter for upstream g (rows, inner): gbase = g * 0 on every
 * written row and g * 1 elsewhere (a multiply, as the reference's mask);
 * gvalues (n, inner) row p = g row idx[p] when p is that row's last writer,
 * zeros otherwise. Either output may be NULL. Replaces the VJP of
 * aops::scatter_dim0 (crates/oxi-autograd/src/ops.rs:531-600). */
int oxi_scatter_rows_bwd(const float* g, int64_t rows, int64_t inner,
                         const int64_t* idx, int64_t n, float* gbase, float* gvalues);
/* Boolean-mask selection over the broadcast of x and mask (strides
 * broadcast-expanded to `shape`): the x values at grid points whose mask value
 * is not zero, in row-major order of `shape`. As in the reference, which marks
 * unpicked points NaN and drops every NaN, a picked NaN of x is dropped too.
 * The output size depends on the data, so the call waits for the device's
 * count of the picks. `*out` holds at least `*count` floats (NULL when none),
 * allocated with oxi_hip_alloc; the caller frees it with oxi_hip_free. By
 * default x is read once: the picks go to a buffer sized for every grid point
 * (moved into one of `*count` floats when they fill at most a third of it),
 * and the call returns once the count is known, while the last picks are
 * still being stored (later calls on the library stream run after them).
 * OXI_MASKED_SELECT_EXACT=1 counts first and allocates exactly `*count`
 * floats, reading x twice. When `record` is not
 * NULL (device memory of oxi_masked_select_record_bytes bytes, 8-byte
 * aligned) it receives the selection's record, one bit per grid point plus
 * per-tile offsets, which oxi_masked_select_bwd reads in place of x and the
 * mask. Replaces Tensor::masked_select (crates/oxi-tensor/src/lib.rs:939-961). */
int oxi_masked_select(const float* x, const int64_t* x_strides,
                      const float* mask, const int64_t* m_strides,
                      const int64_t* shape, int ndim, float** out, int64_t* count,
                      void* record);
/* Bytes of the record of a selection over `shape` (host-side, no device work). */
int oxi_masked_select_record_bytes(const int64_t* shape, int ndim, int64_t* bytes);
/* VJP of oxi_masked_select from its record: grad_x (x_numel floats,
 * row-major of x's own shape) = zeros plus, for each picked grid point in
 * grid order, the next upstream gradient g[k] added at the point's x element,
 * so points that broadcast onto one element accumulate in grid order.
 * `gx_strides` are the row-major strides of x's own shape expanded to `shape`,
 * 0 on the dims where x is broadcast; they are checked against x_numel.
 * `count` is the forward's pick count; a record whose count differs raises
 * the device guard flag (oxi_hip_sync reports it) and no gradient beyond
 * `count` is read. Replaces the VJP of aops::masked_select
 * (crates/oxi-autograd/src/ops.rs:609-667), which walks the mask again. */
int oxi_masked_select_bwd(const void* record, const int64_t* shape, int ndim,
                          const float* g, int64_t count,
                          float* grad_x, const int64_t* gx_strides, int64_t x_numel);

/* ------------------------------------------------------------------------ */
/* Dim reductions.                                                           */

/* Reduce a strided tensor along `dim` into a contiguous output of
 * prod(shape)/shape[dim] floats (row-major over the remaining dims).
 * Semantics of ReduceKind::reduce_strip (crates/oxi-tensor/src/ops.rs:246-285):
 * MAX/MIN ignore NaN (fold with f32::max/min), ARGMAX/ARGMIN keep the first
 * strict winner starting from index 0, indices are written as floats
 * (Tensor::reduce, crates/oxi-tensor/src/lib.rs:519-576). Empty dims: SUM/MEAN/NORM
 * give 0, the others return OXI_INVALID_ARGUMENT. Replaces Tensor::reduce. */
int oxi_reduce(int kind, const float* x, const int64_t* x_strides,
               const int64_t* shape, int ndim, int dim, float* out);

/* ------------------------------------------------------------------------ */
/* Optimizer steps over one flat parameter (n contiguous floats).            */

/* SGD for one parameter: with momentum > 0, buf = momentum*buf + g (buf is
 * updated in place, n floats, zero before the first step) and the update is
 * buf, or g + momentum*buf when `nesterov`; without momentum the update is g
 * and `buf` may be NULL. p_out = p - lr*update; `p_out` may equal `p`.
 * Elementwise f32 in the reference's operation order, so bit-exact with it.
 * Replaces Sgd::step_param (crates/oxi-autograd/src/optim.rs:104-137); the
 * nesterov-without-momentum check of RustSgd::new
 * (crates/oxi-bindings/src/lib.rs:842-846) is repeated here. */
int oxi_sgd_step(const float* p, const float* g, float* buf, float* p_out,
                 int64_t n, float lr, float momentum, int nesterov);
/* Adam / AdamW for one parameter at step t >= 1 (the parameter's own step
 * counter after increment): bias corrections 1 - beta^t in f32 powf; classic
 * Adam (decoupled = 0) adds weight_decay*p to the gradient, AdamW
 * (decoupled = 1) subtracts lr*weight_decay*p after the adaptive step. The
 * moments m, v (n floats each, zero before step 1) are updated in place;
 * `p_out` may equal `p`. Bit-exact with the reference's f32 loop. Replaces
 * AdamW::step_param (crates/oxi-autograd/src/optim.rs:223-262). */
int oxi_adamw_step(const float* p, const float* g, float* m, float* v, float* p_out,
                   int64_t n, float lr, float beta1, float beta2, float eps,
                   float weight_decay, int decoupled, int64_t t);

/* One parameter of a multi-parameter step: its operands as for the
 * single-parameter entry points. Slices must not overlap one another
 * (`p_out` may equal the slice's own `p`). */
typedef struct oxi_sgd_slice {
  const float* p;
  const float* g;
  float* buf; /* NULL allowed when momentum == 0 */
  float* p_out;
  int64_t n;
} oxi_sgd_slice;

typedef struct oxi_adamw_slice {
  const float* p;
  const float* g;
  float* m;
  float* v;
  float* p_out;
  int64_t n;
  int64_t t; /* this parameter's step count, >= 1 */
} oxi_adamw_slice;

/* One optimizer step over a whole parameter list, each slice updated exactly
 * as by oxi_sgd_step / oxi_adamw_step (bit-identical), in few launches: up to
 * 32 slices per launch, their descriptors passed as kernel arguments, so the
 * many small parameters of a model (biases, norm weights) cost no launch of
 * their own. All arguments are checked before anything is launched.
 * Replaces Sgd::step / AdamW::step (crates/oxi-autograd/src/optim.rs:143-148,
 * 267-272) as driven by step_all (crates/oxi-bindings/src/lib.rs:815-826). */
int oxi_sgd_step_multi(const oxi_sgd_slice* slices, int count,
                       float lr, float momentum, int nesterov);
int oxi_adamw_step_multi(const oxi_adamw_slice* slices, int count,
                         float lr, float beta1, float beta2, float eps,
                         float weight_decay, int decoupled);

#ifdef __cplusplus
}
#endif

#endif /* OXIHIP_H */
