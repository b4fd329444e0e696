// RMSNorm and LayerNorm forward/VJP kernels for gfx950.
//
// Layout: x, y, g, dx are contiguous (rows, H) fp32; w, b, dw, db are (H,);
// per-row statistics (mean, rstd) are (rows,). One row group of TPR threads
// owns a row and keeps it in registers (RowTile), so each row crosses HBM once
// per kernel: forward reads x and writes y, backward reads x and g and writes
// dx. Row statistics are reduced with wave64 shuffles (+ LDS across waves).
//
// Parameter gradients (dw = sum_rows g*xhat, db = sum_rows g) are column sums
// over all rows. They are accumulated deterministically: each block owns a
// fixed, strided set of rows, keeps its column partials in registers and
// writes one partial row; a second kernel adds the partial rows in fixed
// order in float64. No float atomics anywhere.
//
// Arithmetic order follows the reference compositions
// (python/oxitorch/nn/functional.py:227-240): mean = sum/H in f32,
// inv = 1/sqrt(var+eps), y = ((x-mu)*inv)*w + b. Row sums are tree-ordered
// rather than the reference's sequential strip sum (ops.rs:256-257).
//
// Norm + activation VJP: when the norm's output y feeds only an activation
// (gelu or silu), the backward takes the activation's upstream gradient g,
// recomputes y from x and the saved statistics with the forward's exact
// arithmetic (no contraction, same operand order, so y is bit-identical),
// forms dy = g * act'(y) with the same functor as the activation's own VJP,
// writes dy (the intermediate's gradient) and continues as the norm VJP.
// Per row that reads x and g and writes dy and dx: 4 row crossings instead
// of the 6 of the two separate VJPs (activation: read y, g, write dy; norm:
// read x, dy, write dx).
#include "norm_bwd.h"

namespace oxi {
namespace {

constexpr int BS = 256;

template <int TPR>
__device__ __forceinline__ float rsum(float v, float* lds) { return group_sum<TPR, float>(v, lds); }
// one barrier per reduction; consecutive reductions alternate slot sets
template <int TPR>
__device__ __forceinline__ float rsum1(float v, float* lds) { return group_sum_once<TPR, float>(v, lds); }

// ---------------------------------------------------------------------------
// Forward, register-resident rows.

// FULL: rows of exactly TPR * NV float4s (H = 4 * TPR * NV), a compile-time
// row length: no padding lanes, no bounds checks.
// NT: threads per block, row_block_threads(TPR) or, for one-wave rows, 1024.
template <int TPR, int NV, bool LN, bool NTS, bool FULL, int NT>
__global__ __launch_bounds__(NT) void norm_fwd_k(const float* __restrict__ x, const float* __restrict__ w,
                                                 const float* __restrict__ b, float* __restrict__ y,
                                                 float* __restrict__ mean, float* __restrict__ rstd,
                                                 int64_t rows, int H_arg, float eps) {
  const int H = FULL ? 4 * TPR * NV : H_arg;
  constexpr int GPB = NT / TPR;
  __shared__ float lds[2 * (NT / 64)];  // mean, then variance
  const int t = threadIdx.x % TPR;
  const int64_t row = (int64_t)blockIdx.x * GPB + threadIdx.x / TPR;
  if (row >= rows) return;  // GPB == 1 whenever TPR > 64: the whole block leaves together
  const int h4 = H >> 2;
  const float fH = (float)H;
  RowTile<TPR, NV> xt;
  xt.load(x + row * H, h4, t);
  float mu = 0.f;
  if constexpr (LN) {
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < NV; ++k) s += (xt.v[k].x + xt.v[k].y) + (xt.v[k].z + xt.v[k].w);
    mu = rsum1<TPR>(s, lds) / fH;
#pragma unroll
    for (int k = 0; k < NV; ++k)
      if (k * TPR + t < h4) xt.v[k] = xt.v[k] - mu;  // centered; padding stays 0
  }
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const f4 v = xt.v[k];
    ss += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
  }
  const float var = rsum1<TPR>(ss, lds + NT / 64) / fH;
  const float inv = 1.0f / sqrtf(var + eps);
  if (t == 0) {
    if (rstd) rstd[row] = inv;
    if (LN && mean) mean[row] = mu;
  }
  const f4* w4 = reinterpret_cast<const f4*>(w);
  const f4* b4 = reinterpret_cast<const f4*>(b);
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int c = k * TPR + t;
    if (c < h4) {
      f4 o = xt.v[k] * inv;
      if (w) o = o * w4[c];
      if (LN && b) o = o + b4[c];
      xt.v[k] = o;
    }
  }
  xt.template store<NTS>(y + row * H, h4, t);
}

// Forward for any H / alignment: one block per row, rows re-read from cache.
template <bool LN>
__global__ __launch_bounds__(BS) void norm_fwd_loop_k(const float* __restrict__ x, const float* __restrict__ w,
                                                      const float* __restrict__ b, float* __restrict__ y,
                                                      float* __restrict__ mean, float* __restrict__ rstd,
                                                      int64_t rows, int H, float eps) {
  __shared__ float lds[BS / 64];
  const int64_t row = blockIdx.x;
  const int t = threadIdx.x;
  const float* xr = x + row * H;
  const float fH = (float)H;
  float mu = 0.f;
  if constexpr (LN) {
    float s = 0.f;
    for (int c = t; c < H; c += BS) s += xr[c];
    mu = rsum<BS>(s, lds) / fH;
  }
  float ss = 0.f;
  for (int c = t; c < H; c += BS) {
    const float v = xr[c] - mu;
    ss += v * v;
  }
  const float var = rsum<BS>(ss, lds) / fH;
  const float inv = 1.0f / sqrtf(var + eps);
  if (t == 0) {
    if (rstd) rstd[row] = inv;
    if (LN && mean) mean[row] = mu;
  }
  float* yr = y + row * H;
  for (int c = t; c < H; c += BS) {
    float o = (xr[c] - mu) * inv;
    if (w) o = o * w[c];
    if (LN && b) o = o + b[c];
    yr[c] = o;
  }
}

// ---------------------------------------------------------------------------
// Host dispatch.

template <bool LN, bool NTS>
void launch_fwd_cfg(int cfg, hipStream_t s, const float* x, const float* w, const float* b, float* y, float* mean,
                    float* rstd, int64_t rows, int h, float eps) {
#define OXI_FWD_NT(TPR, NV, NT)                                                                            \
  if (h == 4 * TPR * NV)                                                                                   \
    norm_fwd_k<TPR, NV, LN, NTS, true, NT><<<dim3((unsigned)ceil_div(rows, NT / TPR)), dim3(NT), 0, s>>>(   \
        x, w, b, y, mean, rstd, rows, h, eps);                                                             \
  else                                                                                                     \
    norm_fwd_k<TPR, NV, LN, NTS, false, NT><<<dim3((unsigned)ceil_div(rows, NT / TPR)), dim3(NT), 0, s>>>(  \
        x, w, b, y, mean, rstd, rows, h, eps);
#define OXI_FWD(TPR, NV)                                                                                   \
  case TPR * 10 + NV:                                                                                      \
    OXI_FWD_NT(TPR, NV, row_block_threads(TPR))                                                            \
    break;
  // One-wave rows: 16 to a block when that leaves at most one block per CU
  // (4096 rows of 768 floats: C1's rms_norm_fwd 6.8 us against 7.3 with 4
  // to a block); with more rows 4 to a block (C5's 16384 rows: 18.4-18.6 us
  // against 19.4-19.7 at 16).
#define OXI_FWD1(NV)                                                                                       \
  case 640 + NV:                                                                                           \
    if (rows <= 16 * (int64_t)cu_count()) {                                                                \
      OXI_FWD_NT(64, NV, 1024)                                                                             \
    } else {                                                                                               \
      OXI_FWD_NT(64, NV, row_block_threads(64))                                                            \
    }                                                                                                      \
    break;
  switch (cfg) {
    OXI_FWD1(1)
    OXI_FWD1(2)
    OXI_FWD1(3)
    OXI_FWD1(4)
    OXI_FWD(256, 2)
    OXI_FWD(256, 4)
    OXI_FWD(512, 2)
    OXI_FWD(256, 8)
    default:
      norm_fwd_loop_k<LN><<<dim3((unsigned)rows), dim3(BS), 0, s>>>(x, w, b, y, mean, rstd, rows, h, eps);
  }
#undef OXI_FWD
#undef OXI_FWD1
#undef OXI_FWD_NT
}

template <bool LN>
int launch_fwd(const float* x, const float* w, const float* b, float* y, float* mean, float* rstd,
               int64_t rows, int64_t H, float eps) {
  hipStream_t s = stream();
  int cfg = vec_ok(H, {x, w, b, y}) ? pick_row_cfg(H / 4) : 0;
#ifdef OXI_NORM_FWD_512X2
  if (cfg == 2564) cfg = 5122;
#endif
  const int h = (int)H;
  if (nt_stores(rows * H * 4)) launch_fwd_cfg<LN, true>(cfg, s, x, w, b, y, mean, rstd, rows, h, eps);
  else launch_fwd_cfg<LN, false>(cfg, s, x, w, b, y, mean, rstd, rows, h, eps);
  return check_launch(LN ? "layer_norm_fwd" : "rms_norm_fwd");
}

// The VJP with activation `act` folded in (OXI_ACT_NONE: the plain VJP),
// launched by the translation unit that instantiates it.
int launch_act_bwd(bool ln, int mode, int act, const NormBwdArgs& a) {
  switch (act) {
    case OXI_ACT_NONE:
      return norm_bwd_none(ln, mode, a);
    case OXI_ACT_GELU_TANH:
    case OXI_ACT_GELU_ERF:
      return norm_bwd_gelu(act, ln, mode, a);
    case OXI_ACT_SILU:
      return norm_bwd_silu(ln, mode, a);
    default:
      return norm_bwd_softmax(act, ln, mode, a);
  }
}

// Whether the leading-dim sum fits the launch: one-wave rows (a wave walks
// a position's rows), rows a multiple of lead.
int lsum_check(const char* what, int64_t lead, int64_t rows, int64_t cols, const float* dx, const float* dx_sum) {
  if (lead < 1 || rows % lead != 0)
    return fail(OXI_INVALID_ARGUMENT, "%s: %lld rows are not a multiple of lead %lld", what, (long long)rows,
                (long long)lead);
  if (lead % LSUM_DEPTH != 0 || rows / lead > ((int64_t)1 << 30))
    return fail(OXI_NOT_IMPLEMENTED, "%s: lead %lld is not a multiple of %d (or positions exceed 2^30); run the VJP "
                "and the reduction", what, (long long)lead, LSUM_DEPTH);
  if (!dx || !dx_sum) return fail(OXI_INVALID_ARGUMENT, "%s: dx and dx_sum must not be NULL", what);
  // dx_sum rows are written as float4s, like dx
  if (!vec_ok(cols, {dx_sum}))
    return fail(OXI_NOT_IMPLEMENTED, "%s: dx_sum at %p is not 16-byte aligned; run the VJP and the reduction", what,
                static_cast<const void*>(dx_sum));
  if (pick_bwd_cfg(cols / 4) / 10 != 64)
    return fail(OXI_NOT_IMPLEMENTED, "%s: rows of %lld floats are wider than one wave; run the VJP and the reduction",
                what, (long long)cols);
  return OXI_OK;
}

// Shared checks of the fused entry points; OXI_OK means "launch".
int check_act(const char* what, int act, int mode, const float* x, const float* w, const float* b, const float* g,
              const float* dyo, const float* dx, int64_t rows, int64_t cols, bool allow_none = false) {
  if ((act < OXI_ACT_GELU_TANH || act > OXI_ACT_LOG_SOFTMAX) && !(allow_none && act == OXI_ACT_NONE))
    return fail(OXI_INVALID_ARGUMENT, "%s: unknown activation %d", what, act);
  if (mode != OXI_NORM_VJP_REF && mode != OXI_NORM_VJP_EXACT)
    return fail(OXI_INVALID_ARGUMENT, "%s: unknown VJP mode %d", what, mode);
  if (rows && cols && !(vec_ok(cols, {x, w, b, g, dyo, dx}) && pick_bwd_cfg(cols / 4)))
    return fail(OXI_NOT_IMPLEMENTED, "%s: rows of %lld floats at these addresses do not vectorize; run the two VJPs",
                what, (long long)cols);
  // the softmax's row sums must follow the softmax kernels' lane layout
  if (rows && cols && is_softmax_act(act) && pick_bwd_cfg(cols / 4) != pick_row_cfg(cols / 4))
    return fail(OXI_NOT_IMPLEMENTED, "%s: softmax rows of %lld floats use another lane layout; run the two VJPs",
                what, (long long)cols);
  return OXI_OK;
}

int check_rows(const char* what, const void* x, const void* y, int64_t rows, int64_t cols) {
  if (rows < 0 || cols < 0) return fail(OXI_INVALID_ARGUMENT, "%s: negative size (%lld, %lld)", what, (long long)rows, (long long)cols);
  if (cols > (int64_t)1 << 30 || rows > ((int64_t)1 << 31) - 1)
    return fail(OXI_INVALID_ARGUMENT, "%s: size (%lld, %lld) exceeds the kernel limits", what, (long long)rows, (long long)cols);
  if ((rows && cols) && (!x || !y)) return fail(OXI_INVALID_ARGUMENT, "%s: NULL tensor pointer", what);
  return OXI_OK;
}

}  // namespace
}  // namespace oxi

using namespace oxi;

extern "C" {

int oxi_rms_norm_fwd(const float* x, const float* w, float* y, float* rstd, int64_t rows, int64_t cols, float eps) {
  if (int rc = check_rows("rms_norm_fwd", x, y, rows, cols)) return rc;
  if (rows == 0) return OXI_OK;
  OXI_CHECK_INIT();
  if (cols == 0) return fail(OXI_INVALID_ARGUMENT, "rms_norm_fwd: cannot normalize a zero-length last dim");
  return launch_fwd<false>(x, w, nullptr, y, nullptr, rstd, rows, cols, eps);
}

int oxi_rms_norm_bwd(const float* x, const float* w, const float* rstd, const float* g, float* dx, float* dw,
                     int64_t rows, int64_t cols, int mode) {
  if (int rc = check_rows("rms_norm_bwd", x, g, rows, cols)) return rc;
  if (!rstd && rows) return fail(OXI_INVALID_ARGUMENT, "rms_norm_bwd: rstd must not be NULL");
  if (mode != OXI_NORM_VJP_REF && mode != OXI_NORM_VJP_EXACT)
    return fail(OXI_INVALID_ARGUMENT, "rms_norm_bwd: unknown VJP mode %d", mode);
  OXI_CHECK_INIT();
  if (rows == 0 || cols == 0) {
    if (dw && cols) return oxi_fill(dw, cols, 0.f);
    return OXI_OK;
  }
  return norm_bwd_none(false, mode, NormBwdArgs{x, w, nullptr, nullptr, rstd, g, nullptr, dx, dw, nullptr, rows, cols});
}

int oxi_layer_norm_fwd(const float* x, const float* w, const float* b, float* y, float* mean, float* rstd,
                       int64_t rows, int64_t cols, float eps) {
  if (int rc = check_rows("layer_norm_fwd", x, y, rows, cols)) return rc;
  if (rows == 0) return OXI_OK;
  OXI_CHECK_INIT();
  if (cols == 0) return fail(OXI_INVALID_ARGUMENT, "layer_norm_fwd: cannot normalize a zero-length last dim");
  return launch_fwd<true>(x, w, b, y, mean, rstd, rows, cols, eps);
}

int oxi_layer_norm_bwd(const float* x, const float* w, const float* mean, const float* rstd, const float* g,
                       float* dx, float* dw, float* db, int64_t rows, int64_t cols, int mode) {
  if (int rc = check_rows("layer_norm_bwd", x, g, rows, cols)) return rc;
  if ((!rstd || !mean) && rows) return fail(OXI_INVALID_ARGUMENT, "layer_norm_bwd: mean/rstd must not be NULL");
  if (mode != OXI_NORM_VJP_REF && mode != OXI_NORM_VJP_EXACT)
    return fail(OXI_INVALID_ARGUMENT, "layer_norm_bwd: unknown VJP mode %d", mode);
  OXI_CHECK_INIT();
  if (rows == 0 || cols == 0) {
    int rc = OXI_OK;
    if (dw && cols) rc = oxi_fill(dw, cols, 0.f);
    if (!rc && db && cols) rc = oxi_fill(db, cols, 0.f);
    return rc;
  }
  return norm_bwd_none(true, mode, NormBwdArgs{x, w, nullptr, mean, rstd, g, nullptr, dx, dw, db, rows, cols});
}

int oxi_layer_norm_bwd_noalloc(const float* x, const float* w, const float* mean, const float* rstd, const float* g,
                               float* dx, float* dw, float* db, int64_t rows, int64_t cols, int mode) {
  if (int rc = check_rows("layer_norm_bwd_noalloc", x, g, rows, cols)) return rc;
  if ((!rstd || !mean) && rows)
    return fail(OXI_INVALID_ARGUMENT, "layer_norm_bwd_noalloc: mean/rstd must not be NULL");
  if (mode != OXI_NORM_VJP_REF && mode != OXI_NORM_VJP_EXACT)
    return fail(OXI_INVALID_ARGUMENT, "layer_norm_bwd_noalloc: unknown VJP mode %d", mode);
  // initialisation allocates (streams, flags): it must have happened already
  if (!initialised())
    return fail(OXI_INVALID_ARGUMENT, "layer_norm_bwd_noalloc: the library is not initialised; call oxi_hip_init "
                                      "first (this entry point allocates nothing, initialisation does)");
  if (rows == 0 || cols == 0) {
    int rc = OXI_OK;
    if (dw && cols) rc = oxi_fill(dw, cols, 0.f);
    if (!rc && db && cols) rc = oxi_fill(db, cols, 0.f);
    return rc;
  }
  const int cfg = vec_ok(cols, {x, w, g, dx}) ? pick_bwd_cfg(cols / 4) : 0;
  const size_t need = bwd_part_bytes(dw || db, rows, cols, cfg);
  if (need > (size_t)OXI_NOALLOC_SCRATCH_BYTES)
    return fail(OXI_INVALID_ARGUMENT,
                "layer_norm_bwd_noalloc: rows of %lld floats need %zu bytes of scratch for the column partials, "
                "above the fixed %zu bytes; use oxi_layer_norm_bwd",
                (long long)cols, need, (size_t)OXI_NOALLOC_SCRATCH_BYTES);
  void* sp = noalloc_scratch();
  if (!sp) return fail(OXI_OTHER, "layer_norm_bwd_noalloc: no scratch address for the bound device");
  std::lock_guard<std::mutex> lk(noalloc_mutex());
  return norm_bwd_none(true, mode, NormBwdArgs{x, w, nullptr, mean, rstd, g, nullptr, dx, dw, db, rows, cols, sp,
                                               nullptr, 0, (size_t)OXI_NOALLOC_SCRATCH_BYTES});
}

int oxi_rms_norm_bwd_lead_sum(const float* x, const float* w, const float* rstd, const float* g, int act, float* dy,
                              float* dx, float* dw, float* dx_sum, int64_t lead, int64_t rows, int64_t cols,
                              int mode) {
  if (int rc = check_rows("rms_norm_bwd_lead_sum", x, g, rows, cols)) return rc;
  if (!rstd && rows) return fail(OXI_INVALID_ARGUMENT, "rms_norm_bwd_lead_sum: rstd must not be NULL");
  if (int rc = check_act("rms_norm_bwd_lead_sum", act, mode, x, w, nullptr, g, dy, dx, rows, cols, true)) return rc;
  if (rows == 0 || cols == 0) return fail(OXI_NOT_IMPLEMENTED, "rms_norm_bwd_lead_sum: empty rows; run the VJP");
  if (int rc = lsum_check("rms_norm_bwd_lead_sum", lead, rows, cols, dx, dx_sum)) return rc;
  OXI_CHECK_INIT();
  return launch_act_bwd(false, mode, act, NormBwdArgs{x, w, nullptr, nullptr, rstd, g, dy, dx, dw, nullptr, rows, cols, nullptr, dx_sum, lead});
}

int oxi_layer_norm_bwd_lead_sum(const float* x, const float* w, const float* b, const float* mean, const float* rstd,
                                const float* g, int act, float* dy, float* dx, float* dw, float* db, float* dx_sum,
                                int64_t lead, int64_t rows, int64_t cols, int mode) {
  if (int rc = check_rows("layer_norm_bwd_lead_sum", x, g, rows, cols)) return rc;
  if ((!rstd || !mean) && rows)
    return fail(OXI_INVALID_ARGUMENT, "layer_norm_bwd_lead_sum: mean/rstd must not be NULL");
  if (int rc = check_act("layer_norm_bwd_lead_sum", act, mode, x, w, b, g, dy, dx, rows, cols, true)) return rc;
  if (rows == 0 || cols == 0) return fail(OXI_NOT_IMPLEMENTED, "layer_norm_bwd_lead_sum: empty rows; run the VJP");
  if (int rc = lsum_check("layer_norm_bwd_lead_sum", lead, rows, cols, dx, dx_sum)) return rc;
  OXI_CHECK_INIT();
  return launch_act_bwd(true, mode, act, NormBwdArgs{x, w, b, mean, rstd, g, dy, dx, dw, db, rows, cols, nullptr, dx_sum, lead});
}

int oxi_rms_norm_act_bwd(const float* x, const float* w, const float* rstd, const float* g, int act, float* dy,
                         float* dx, float* dw, int64_t rows, int64_t cols, int mode) {
  if (int rc = check_rows("rms_norm_act_bwd", x, g, rows, cols)) return rc;
  if (!rstd && rows) return fail(OXI_INVALID_ARGUMENT, "rms_norm_act_bwd: rstd must not be NULL");
  if (int rc = check_act("rms_norm_act_bwd", act, mode, x, w, nullptr, g, dy, dx, rows, cols)) return rc;
  OXI_CHECK_INIT();
  if (rows == 0 || cols == 0) {
    if (dw && cols) return oxi_fill(dw, cols, 0.f);
    return OXI_OK;
  }
  return launch_act_bwd(false, mode, act, NormBwdArgs{x, w, nullptr, nullptr, rstd, g, dy, dx, dw, nullptr, rows, cols});
}

int oxi_layer_norm_act_bwd(const float* x, const float* w, const float* b, const float* mean, const float* rstd,
                           const float* g, int act, float* dy, float* dx, float* dw, float* db, int64_t rows,
                           int64_t cols, int mode) {
  if (int rc = check_rows("layer_norm_act_bwd", x, g, rows, cols)) return rc;
  if ((!rstd || !mean) && rows) return fail(OXI_INVALID_ARGUMENT, "layer_norm_act_bwd: mean/rstd must not be NULL");
  if (int rc = check_act("layer_norm_act_bwd", act, mode, x, w, b, g, dy, dx, rows, cols)) return rc;
  OXI_CHECK_INIT();
  if (rows == 0 || cols == 0) {
    int rc = OXI_OK;
    if (dw && cols) rc = oxi_fill(dw, cols, 0.f);
    if (!rc && db && cols) rc = oxi_fill(db, cols, 0.f);
    return rc;
  }
  return launch_act_bwd(true, mode, act, NormBwdArgs{x, w, b, mean, rstd, g, dy, dx, dw, db, rows, cols});
}

}  // extern "C"
