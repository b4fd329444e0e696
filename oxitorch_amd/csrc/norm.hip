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
#include "internal.h"
#include "rowtile.h"

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

template <int TPR, int NV, bool LN, bool NTS>
__global__ __launch_bounds__((row_block_threads(TPR))) void norm_fwd_k(const float* __restrict__ x, const float* __restrict__ w,
                                                 const float* __restrict__ b, float* __restrict__ y,
                                                 float* __restrict__ mean, float* __restrict__ rstd,
                                                 int64_t rows, int H, float eps) {
  constexpr int NT = row_block_threads(TPR);
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
// Backward, register-resident rows, grid-strided over rows, column partials.
//
// part (if not null): [2][gridDim.x][H] floats, dw partials then db partials.

// Threads per backward block: one-wave rows run 16 to a block (one block per
// CU: 16 waves in flight, one partial row per CU), or 8 to a block (two
// blocks per CU) when 4 float4s per lane would not fit the registers of 16;
// wider rows 1 per block.
template <int TPR, int NV>
constexpr int bwd_threads() { return TPR == 64 ? (NV <= 3 ? 1024 : 512) : BS; }

template <int TPR, int NV, int MODE, bool LN, bool NTS>
__global__ __launch_bounds__((bwd_threads<TPR, NV>())) void norm_bwd_k(const float* __restrict__ x, const float* __restrict__ w,
                                                 const float* __restrict__ mean, const float* __restrict__ rstd,
                                                 const float* __restrict__ g, float* __restrict__ dx,
                                                 float* __restrict__ part, int64_t rows, int H) {
  constexpr int NT = bwd_threads<TPR, NV>();
  constexpr int GPB = NT / TPR;
  constexpr int ROWF = TPR * NV * 4;  // floats a group covers
  __shared__ float lds[2 * (BS / 64)];
  __shared__ float comb[GPB > 1 ? GPB * ROWF : 1];
  const int t = threadIdx.x % TPR;
  const int gi = threadIdx.x / TPR;
  const int h4 = H >> 2;
  const float fH = (float)H;
  const float inv_n = 1.0f / fH;
  const f4* w4 = reinterpret_cast<const f4*>(w);
  const f4 zero = {0.f, 0.f, 0.f, 0.f};
  f4 pdw[NV], pdb[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) { pdw[k] = zero; pdb[k] = zero; }

  // weights (padding lanes: 0); cached, re-read per row to save registers
  auto wv_at = [&](int k) -> f4 {
    const int c = k * TPR + t;
    return (c < h4) ? (w ? w4[c] : f4{1.f, 1.f, 1.f, 1.f}) : zero;
  };
  // rows are double-buffered: the next row's x, g and statistics are in
  // flight while the current row is reduced and stored
  const int64_t ngroups = (int64_t)gridDim.x * GPB;
  int64_t row = (int64_t)blockIdx.x * GPB + gi;
  int red = 0;  // reductions so far: consecutive ones use alternate LDS slot sets
  auto slot = [&]() { return lds + ((red++ & 1) ? BS / 64 : 0); };
  RowTile<TPR, NV> xt, gt;
  float inv = 0.f, mu = 0.f;
  if (row < rows) {
    xt.load(x + row * H, h4, t);
    gt.load(g + row * H, h4, t);
    inv = rstd[row];
    if constexpr (LN) mu = mean[row];
  }
  while (row < rows) {
    const int64_t nrow = row + ngroups;
    RowTile<TPR, NV> xn, gn;
    float ninv = 0.f, nmu = 0.f;
    if (nrow < rows) {
      xn.load(x + nrow * H, h4, t);
      gn.load(g + nrow * H, h4, t);
      ninv = rstd[nrow];
      if constexpr (LN) nmu = mean[nrow];
    }
    // xhat = (x - mu) * inv ; gw = g * w   (padding lanes stay 0)
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int c = k * TPR + t;
      f4 xh = LN ? (xt.v[k] - mu) * inv : xt.v[k] * inv;
      if (c >= h4) xh = zero;
      xt.v[k] = xh;  // xt now holds xhat
      pdw[k] = pdw[k] + gt.v[k] * xh;
      if constexpr (LN) pdb[k] = pdb[k] + gt.v[k];
    }
    if (dx) {
      if constexpr (MODE == OXI_NORM_VJP_REF) {
        // gc = (g*w)*inv ; LN: dx = gc + (-sum(gc)) * (1/H)   (mean VJP, ops.rs:342-347)
        float s = 0.f;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
          gt.v[k] = (gt.v[k] * wv_at(k)) * inv;
          s += (gt.v[k].x + gt.v[k].y) + (gt.v[k].z + gt.v[k].w);
        }
        if constexpr (LN) {
          const float corr = (-rsum1<TPR>(s, slot())) * inv_n;
#pragma unroll
          for (int k = 0; k < NV; ++k) gt.v[k] = gt.v[k] + corr;
        }
      } else {
        // exact: RMS dx = (gw - xhat*mean(gw*xhat))*inv ; LN also subtracts mean(gw)
        float sa = 0.f, sb = 0.f;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
          gt.v[k] = gt.v[k] * wv_at(k);
          const f4 p = gt.v[k] * xt.v[k];
          sb += (p.x + p.y) + (p.z + p.w);
          sa += (gt.v[k].x + gt.v[k].y) + (gt.v[k].z + gt.v[k].w);
        }
        float a = 0.f;
        if constexpr (LN) a = rsum1<TPR>(sa, slot()) * inv_n;
        const float bcoef = rsum1<TPR>(sb, slot()) * inv_n;
#pragma unroll
        for (int k = 0; k < NV; ++k) gt.v[k] = ((gt.v[k] - a) - xt.v[k] * bcoef) * inv;
      }
      gt.template store<NTS>(dx + row * H, h4, t);
    }
    xt = xn;
    gt = gn;
    inv = ninv;
    mu = nmu;
    row = nrow;
  }
  if (!part) return;
  float* pw = part + (int64_t)blockIdx.x * H;
  float* pb = part + ((int64_t)gridDim.x + blockIdx.x) * H;
  if constexpr (GPB == 1) {
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int c = k * TPR + t;
      if (c < h4) {
        reinterpret_cast<f4*>(pw)[c] = pdw[k];
        if (LN) reinterpret_cast<f4*>(pb)[c] = pdb[k];
      }
    }
  } else {
    // combine the GPB groups of this block in fixed group order, one plane
    // (dw, then db) at a time through the same LDS buffer
#pragma unroll
    for (int plane = 0; plane < (LN ? 2 : 1); ++plane) {
#pragma unroll
      for (int k = 0; k < NV; ++k) reinterpret_cast<f4*>(comb + gi * ROWF)[k * TPR + t] = plane ? pdb[k] : pdw[k];
      __syncthreads();
      float* dst = plane ? pb : pw;
      for (int c = threadIdx.x; c < H; c += NT) {
        float sum = comb[c];
#pragma unroll
        for (int q = 1; q < GPB; ++q) sum += comb[q * ROWF + c];
        dst[c] = sum;
      }
      __syncthreads();
    }
  }
}

// Backward for any H / alignment: each block loops over its rows; the block's
// partial row lives in global memory owned by that block alone.
template <int MODE, bool LN>
__global__ __launch_bounds__(BS) void norm_bwd_loop_k(const float* __restrict__ x, const float* __restrict__ w,
                                                      const float* __restrict__ mean, const float* __restrict__ rstd,
                                                      const float* __restrict__ g, float* __restrict__ dx,
                                                      float* __restrict__ part, int64_t rows, int H) {
  __shared__ float lds[2 * (BS / 64)];
  const int t = threadIdx.x;
  const float fH = (float)H;
  const float inv_n = 1.0f / fH;
  float* pw = part ? part + (int64_t)blockIdx.x * H : nullptr;
  float* pb = part ? part + ((int64_t)gridDim.x + blockIdx.x) * H : nullptr;
  if (part)
    for (int c = t; c < H; c += BS) { pw[c] = 0.f; if (LN) pb[c] = 0.f; }
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const float* xr = x + row * H;
    const float* gr = g + row * H;
    const float inv = rstd[row];
    const float mu = LN ? mean[row] : 0.f;
    float sa = 0.f, sb = 0.f;
    for (int c = t; c < H; c += BS) {
      const float xh = (xr[c] - mu) * inv;
      const float gv = gr[c];
      const float gw = w ? gv * w[c] : gv;
      if (part) { pw[c] += gv * xh; if (LN) pb[c] += gv; }
      if (MODE == OXI_NORM_VJP_REF) sa += gw * inv;
      else { sa += gw; sb += gw * xh; }
    }
    if (!dx) continue;
    float a = 0.f, bc = 0.f;
    if (MODE == OXI_NORM_VJP_REF) {
      if (LN) a = (-rsum<BS>(sa, lds)) * inv_n;
    } else {
      if (LN) a = rsum<BS>(sa, lds) * inv_n;
      bc = rsum<BS>(sb, lds + BS / 64) * inv_n;
    }
    float* dr = dx + row * H;
    for (int c = t; c < H; c += BS) {
      const float gv = gr[c];
      const float gw = w ? gv * w[c] : gv;
      if (MODE == OXI_NORM_VJP_REF) {
        dr[c] = (gw * inv) + a;
      } else {
        const float xh = (xr[c] - mu) * inv;
        dr[c] = ((gw - a) - xh * bc) * inv;
      }
    }
  }
}

// out[c] = sum over partial rows b (fixed order, float64) of part[b][c].
// A block owns 64 columns; its FIN_W waves each sum the rows b = s, s+FIN_W,
// ... of one slice s (FIN_U loads in flight), then the slice sums are added
// in slice order. blockIdx.y selects the dw (0) or db (1) plane.
constexpr int FIN_W = 16;
constexpr int FIN_U = 16;

__global__ __launch_bounds__(64 * FIN_W) void col_finish_k(const float* __restrict__ part, int nb, int H,
                                                           float* __restrict__ out0, float* __restrict__ out1) {
  float* out = blockIdx.y ? out1 : out0;
  if (!out) return;
  const float* p = part + (int64_t)blockIdx.y * nb * H;
  const int lane = threadIdx.x & 63;
  const int slice = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + lane;
  const int cc = min(c, H - 1);  // in range: loads issue together
  double acc = 0.0;
  for (int b0 = slice; b0 < nb; b0 += FIN_W * FIN_U) {
    float v[FIN_U];
#pragma unroll
    for (int q = 0; q < FIN_U; ++q) v[q] = p[(int64_t)min(b0 + FIN_W * q, nb - 1) * H + cc];
#pragma unroll
    for (int q = 0; q < FIN_U; ++q)
      if (b0 + FIN_W * q < nb) acc += (double)v[q];
  }
  __shared__ double s[FIN_W][64];
  s[slice][lane] = acc;
  __syncthreads();
  if (slice == 0 && c < H) {
    double t = s[0][lane];
#pragma unroll
    for (int i = 1; i < FIN_W; ++i) t += s[i][lane];
    out[c] = (float)t;
  }
}

// ---------------------------------------------------------------------------
// Host dispatch.

bool vec_ok(int64_t H, std::initializer_list<const void*> ptrs) {
  if (H % 4 != 0) return false;
  for (const void* p : ptrs)
    if (p && (reinterpret_cast<uintptr_t>(p) & 15u)) return false;
  return true;
}

// (TPR, NV) of the backward for a vectorized row of h4 float4s; 0 when it
// does not fit. The backward keeps its rows multi-float4 per lane: it walks
// rows grid-strided with column partials, and one-wave groups let 16 rows
// share a block.
int pick_bwd_cfg(int64_t h4) {
  if (h4 <= 64) return 641;
  if (h4 <= 128) return 642;
  if (h4 <= 192) return 643;
  if (h4 <= 256) return 644;
  if (h4 <= 512) return 2562;
  if (h4 <= 1024) return 2564;
  if (h4 <= 2048) return 2568;
  return 0;
}

template <bool LN, bool NTS>
void launch_fwd_cfg(int cfg, hipStream_t s, const float* x, const float* w, const float* b, float* y, float* mean,
                    float* rstd, int64_t rows, int h, float eps) {
#define OXI_FWD(TPR, NV)                                                                                   \
  case TPR * 10 + NV:                                                                                      \
    norm_fwd_k<TPR, NV, LN, NTS><<<dim3((unsigned)ceil_div(rows, row_block_threads(TPR) / TPR)),          \
                                   dim3(row_block_threads(TPR)), 0, s>>>(x, w, b, y, mean, rstd, rows, h, eps); \
    break;
  switch (cfg) {
    OXI_FWD(64, 1)
    OXI_FWD(64, 2)
    OXI_FWD(64, 3)
    OXI_FWD(64, 4)
    OXI_FWD(256, 2)
    OXI_FWD(256, 4)
    OXI_FWD(256, 8)
    default:
      norm_fwd_loop_k<LN><<<dim3((unsigned)rows), dim3(BS), 0, s>>>(x, w, b, y, mean, rstd, rows, h, eps);
  }
#undef OXI_FWD
}

template <bool LN>
int launch_fwd(const float* x, const float* w, const float* b, float* y, float* mean, float* rstd,
               int64_t rows, int64_t H, float eps) {
  hipStream_t s = stream();
  const int cfg = vec_ok(H, {x, w, b, y}) ? pick_row_cfg(H / 4) : 0;
  const int h = (int)H;
  if (nt_stores(rows * H * 4)) launch_fwd_cfg<LN, true>(cfg, s, x, w, b, y, mean, rstd, rows, h, eps);
  else launch_fwd_cfg<LN, false>(cfg, s, x, w, b, y, mean, rstd, rows, h, eps);
  return check_launch(LN ? "layer_norm_fwd" : "rms_norm_fwd");
}

template <bool LN, int MODE, bool NTS>
void launch_bwd_cfg(int cfg, hipStream_t s, int64_t nblk, int nt, const float* x, const float* w, const float* mean,
                    const float* rstd, const float* g, float* dx, float* part, int64_t rows, int h) {
#define OXI_BWD(TPR, NV)                                                                                   \
  case TPR * 10 + NV:                                                                                      \
    norm_bwd_k<TPR, NV, MODE, LN, NTS><<<dim3((unsigned)nblk), dim3(nt), 0, s>>>(x, w, mean, rstd, g, dx,  \
                                                                                part, rows, h);            \
    break;
  switch (cfg) {
    OXI_BWD(64, 1)
    OXI_BWD(64, 2)
    OXI_BWD(64, 3)
    OXI_BWD(64, 4)
    OXI_BWD(256, 2)
    OXI_BWD(256, 4)
    OXI_BWD(256, 8)
    default:
      norm_bwd_loop_k<MODE, LN><<<dim3((unsigned)nblk), dim3(BS), 0, s>>>(x, w, mean, rstd, g, dx, part, rows, h);
  }
#undef OXI_BWD
}

template <bool LN, int MODE>
int launch_bwd(const float* x, const float* w, const float* mean, const float* rstd, const float* g,
               float* dx, float* dw, float* db, int64_t rows, int64_t H) {
  hipStream_t s = stream();
  const bool need_part = dw || (LN && db);
  const int cfg = vec_ok(H, {x, w, g, dx}) ? pick_bwd_cfg(H / 4) : 0;
  const int tpr = cfg ? cfg / 10 : BS;
  const int nt = tpr == 64 ? (cfg % 10 <= 3 ? 1024 : 512) : BS;  // bwd_threads<TPR, NV>()
  const int gpb = nt / tpr;
  // Blocks: enough to fill the chip, few enough that the partial rows stay
  // a small fraction of the row traffic.
  int64_t nblk = ceil_div(rows, gpb);
  // (measured: 2 blocks per CU beat 3 and 4 for 4096-float rows)
  const int64_t cap = (int64_t)cu_count() * (nt == 1024 ? 1 : 2);
  if (need_part && nblk > cap) nblk = cap;
  if (!need_part && nblk > (int64_t)cu_count() * 16) nblk = (int64_t)cu_count() * 16;
  if (nblk < 1) nblk = 1;
  Workspace ws(need_part ? sizeof(float) * 2 * (size_t)nblk * (size_t)H : 0);
  if (need_part && !ws.p) return OXI_OTHER;
  float* part = ws.as<float>();
  const int h = (int)H;
  if (nt_stores(rows * H * 4)) launch_bwd_cfg<LN, MODE, true>(cfg, s, nblk, nt, x, w, mean, rstd, g, dx, part, rows, h);
  else launch_bwd_cfg<LN, MODE, false>(cfg, s, nblk, nt, x, w, mean, rstd, g, dx, part, rows, h);
  int rc = check_launch(LN ? "layer_norm_bwd" : "rms_norm_bwd");
  if (rc != OXI_OK) return rc;
  if (need_part) {
    col_finish_k<<<dim3((unsigned)ceil_div(H, 64), LN ? 2 : 1), dim3(64 * FIN_W), 0, s>>>(part, (int)nblk, h, dw,
                                                                                    LN ? db : nullptr);
    rc = check_launch("norm_param_grad_finish");
  }
  return rc;
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
  return mode == OXI_NORM_VJP_REF
             ? launch_bwd<false, OXI_NORM_VJP_REF>(x, w, nullptr, rstd, g, dx, dw, nullptr, rows, cols)
             : launch_bwd<false, OXI_NORM_VJP_EXACT>(x, w, nullptr, rstd, g, dx, dw, nullptr, rows, cols);
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
  return mode == OXI_NORM_VJP_REF
             ? launch_bwd<true, OXI_NORM_VJP_REF>(x, w, mean, rstd, g, dx, dw, db, rows, cols)
             : launch_bwd<true, OXI_NORM_VJP_EXACT>(x, w, mean, rstd, g, dx, dw, db, rows, cols);
}

}  // extern "C"
