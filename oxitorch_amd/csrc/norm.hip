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
#include "internal.h"
#include "ops.h"
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
constexpr int bwd_threads() { return TPR == 64 ? (NV <= 3 ? 1024 : 512) : TPR; }

// ACT_NONE: g is the norm output's gradient. Otherwise g is the gradient of
// act(y) and the kernel first forms dy (written to dyo if set): g * act'(y)
// for the elementwise activations, the softmax VJP over the row for
// OXI_ACT_SOFTMAX / OXI_ACT_LOG_SOFTMAX.
constexpr int ACT_NONE = -1;
constexpr bool is_softmax_act(int act) { return act == OXI_ACT_SOFTMAX || act == OXI_ACT_LOG_SOFTMAX; }

template <int ACT>
__device__ __forceinline__ float act_vjp(float y, float g) {
  if constexpr (ACT == OXI_ACT_GELU_TANH) return GeluTanhBwd{}(y, g);
  else if constexpr (ACT == OXI_ACT_GELU_ERF) return GeluErfBwd{}(y, g);
  else return SiluBwd{}(y, g);
}

template <int TPR, int NV, int MODE, bool LN, bool NTS, int ACT>
__global__ __launch_bounds__((bwd_threads<TPR, NV>())) void norm_bwd_k(const float* __restrict__ x, const float* __restrict__ w,
                                                 const float* __restrict__ b,
                                                 const float* __restrict__ mean, const float* __restrict__ rstd,
                                                 const float* __restrict__ g, float* __restrict__ dyo,
                                                 float* __restrict__ dx,
                                                 float* __restrict__ part, int64_t rows, int H) {
  constexpr int NT = bwd_threads<TPR, NV>();
  constexpr int GPB = NT / TPR;
  constexpr int ROWF = TPR * NV * 4;  // floats a group covers
  __shared__ float lds[2 * (NT / 64)];
  __shared__ float comb[GPB > 1 ? GPB * ROWF : 1];
  const int t = threadIdx.x % TPR;
  const int gi = threadIdx.x / TPR;
  const int h4 = H >> 2;
  const float fH = (float)H;
  const float inv_n = 1.0f / fH;
  const f4* w4 = reinterpret_cast<const f4*>(w);
  const f4* b4 = reinterpret_cast<const f4*>(b);
  const f4 zero = {0.f, 0.f, 0.f, 0.f};
  f4 pdw[NV], pdb[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) { pdw[k] = zero; pdb[k] = zero; }

  // Wide rows (TPR > 64) keep the loop-invariant weights (and, for the
  // activation prologue, biases) in registers: a load inside the row loop is
  // younger than the next row's prefetch, and the in-order vmcnt wait for it
  // also waits for the prefetch. One-wave rows run 16 waves to a CU at up to
  // 128 VGPRs, where those registers cost more than the wait: they re-read
  // w and b (cached) per row. Padding lanes (c >= h4) are zeroed at use.
  constexpr bool REG_W = TPR > 64;
  f4 wr[NV], br[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int cc = min(k * TPR + t, h4 - 1);
    wr[k] = (REG_W && w) ? w4[cc] : f4{1.f, 1.f, 1.f, 1.f};
    br[k] = (REG_W && ACT != ACT_NONE && LN && b) ? b4[cc] : zero;
  }
  auto wv_at = [&](int k) -> f4 {
    const int c = k * TPR + t;
    if constexpr (REG_W) return c < h4 ? wr[k] : zero;
    else return c < h4 ? (w ? w4[c] : f4{1.f, 1.f, 1.f, 1.f}) : zero;
  };

  // Rows are double-buffered: the next row's x, g and statistics are in
  // flight while the current row is reduced and stored. For wide rows the
  // two register sets swap roles every row (the loop is unrolled twice, so
  // no copies) and every prefetch load issues (row and column clamped in
  // bounds), so the wait before a row's first use counts exactly the
  // younger loads.
  const int64_t ngroups = (int64_t)gridDim.x * GPB;
  int64_t row = (int64_t)blockIdx.x * GPB + gi;
  int red = 0;  // reductions so far: consecutive ones use alternate LDS slot sets
  auto slot = [&]() { return lds + ((red++ & 1) ? NT / 64 : 0); };
  auto fetch = [&](RowTile<TPR, NV>& xt, RowTile<TPR, NV>& gt, float& inv, float& mu, int64_t r) {
    r = r < rows ? r : rows - 1;
    xt.load_clamped(x + r * H, h4, t);
    gt.load_clamped(g + r * H, h4, t);
    inv = rstd[r];
    if constexpr (LN) mu = mean[r];
  };
  auto process = [&](RowTile<TPR, NV>& xt, RowTile<TPR, NV>& gt, const float inv, const float mu, const int64_t r) {
    if constexpr (is_softmax_act(ACT)) {
      // p = softmax(y) (or log_softmax) as sm_fwd_k forms it over the same
      // lane layout, then dy = p * (g - sum(g*p)) (log: g - exp(p) * sum(g))
      // as sm_bwd_k does; padding lanes (c >= h4) hold 0 in g and in exp(y).
      constexpr bool LOG = ACT == OXI_ACT_LOG_SOFTMAX;
      f4 pk[NV];
      float m = NEG_INF;
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        pk[k] = zero;
        const int c = k * TPR + t;
        if (c < h4) {
          f4 yv = LN ? (xt.v[k] - mu) * inv : xt.v[k] * inv;
          if (w) yv = yv * (REG_W ? wr[k] : w4[c]);
          if (LN && b) yv = yv + (REG_W ? br[k] : b4[c]);
          pk[k] = yv;
          m = fmaxf(m, max4(yv));
        } else {
          gt.v[k] = zero;
        }
      }
      m = group_max_once<TPR>(m, slot());
      float s = 0.f;
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        if (k * TPR + t < h4) {
          const f4 z = pk[k] - m;
          const f4 e = exp4(z);
          s += sum4(e);
          pk[k] = LOG ? z : e;
        }
      }
      s = rsum1<TPR>(s, slot());
      if constexpr (LOG) {
        const float L = logf(s);
#pragma unroll
        for (int k = 0; k < NV; ++k) pk[k] = pk[k] - L;
      } else {
#pragma unroll
        for (int k = 0; k < NV; ++k) pk[k] = pk[k] / s;
      }
      float sg = 0.f;
#pragma unroll
      for (int k = 0; k < NV; ++k) sg += LOG ? sum4(gt.v[k]) : sum4(gt.v[k] * pk[k]);
      sg = rsum1<TPR>(sg, slot());
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        if constexpr (LOG) gt.v[k] = gt.v[k] - exp4(pk[k]) * sg;
        else gt.v[k] = pk[k] * (gt.v[k] - sg);
      }
      if (dyo) gt.template store<NTS>(dyo + r * H, h4, t);
    } else if constexpr (ACT != ACT_NONE) {
      // y as the forward wrote it, then dy = g * act'(y)   (padding lanes: 0)
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        if (k * TPR + t < h4) {
          const int c = k * TPR + t;
          f4 yv = LN ? (xt.v[k] - mu) * inv : xt.v[k] * inv;
          if (w) yv = yv * (REG_W ? wr[k] : w4[c]);
          if (LN && b) yv = yv + (REG_W ? br[k] : b4[c]);
          const f4 gv = gt.v[k];
          gt.v[k] = f4{act_vjp<ACT>(yv.x, gv.x), act_vjp<ACT>(yv.y, gv.y), act_vjp<ACT>(yv.z, gv.z),
                       act_vjp<ACT>(yv.w, gv.w)};
        } else {
          gt.v[k] = zero;
        }
      }
      if (dyo) gt.template store<NTS>(dyo + r * H, h4, t);
    }
    // xhat = (x - mu) * inv ; gw = g * w   (padding lanes: 0)
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int c = k * TPR + t;
      f4 xh = LN ? (xt.v[k] - mu) * inv : xt.v[k] * inv;
      if (c >= h4) {
        xh = zero;
        gt.v[k] = zero;
      }
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
      gt.template store<NTS>(dx + r * H, h4, t);
    }
  };
  RowTile<TPR, NV> xa, ga, xb, gb;
  float ia = 0.f, ma = 0.f, ib = 0.f, mb = 0.f;
  if constexpr (!REG_W) {
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
      process(xt, gt, inv, mu, row);
      xt = xn;
      gt = gn;
      inv = ninv;
      mu = nmu;
      row = nrow;
    }
  } else {
    // The scheduling barriers keep the current row's first use below the next
    // row's loads, so its wait leaves those loads in flight.
    fetch(xa, ga, ia, ma, row);
    while (row < rows) {
      fetch(xb, gb, ib, mb, row + ngroups);
      __builtin_amdgcn_sched_barrier(0);
      process(xa, ga, ia, ma, row);
      row += ngroups;
      if (row >= rows) break;
      fetch(xa, ga, ia, ma, row + ngroups);
      __builtin_amdgcn_sched_barrier(0);
      process(xb, gb, ib, mb, row);
      row += ngroups;
    }
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
// share a block. Rows past 2048 floats spread over 512 threads: the norm +
// activation VJP needs 218 VGPRs at 256 x 4 float4s (2 waves per SIMD) and
// 128 at 512 x 2 (4 waves per SIMD), and the plain VJP runs as fast at either
// width, so both use the same configuration and their row sums agree bit
// for bit.
int pick_bwd_cfg(int64_t h4) {
  if (h4 <= 64) return 641;
  if (h4 <= 128) return 642;
  if (h4 <= 192) return 643;
  if (h4 <= 256) return 644;
  if (h4 <= 512) return 2562;
  if (h4 <= 1024) return 5122;
  if (h4 <= 2048) return 5124;
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

template <bool LN, int MODE, bool NTS, int ACT>
void launch_bwd_cfg(int cfg, hipStream_t s, int64_t nblk, int nt, const float* x, const float* w, const float* b,
                    const float* mean, const float* rstd, const float* g, float* dyo, float* dx, float* part,
                    int64_t rows, int h) {
#define OXI_BWD(TPR, NV)                                                                                   \
  case TPR * 10 + NV:                                                                                      \
    norm_bwd_k<TPR, NV, MODE, LN, NTS, ACT><<<dim3((unsigned)nblk), dim3(nt), 0, s>>>(                     \
        x, w, b, mean, rstd, g, dyo, dx, part, rows, h);                                                   \
    break;
  switch (cfg) {
    OXI_BWD(64, 1)
    OXI_BWD(64, 2)
    OXI_BWD(64, 3)
    OXI_BWD(64, 4)
    OXI_BWD(256, 2)
    OXI_BWD(512, 2)
    OXI_BWD(512, 4)
    default:
      // vectorized shapes only when fused (the entry point checks)
      if constexpr (ACT == ACT_NONE)
        norm_bwd_loop_k<MODE, LN><<<dim3((unsigned)nblk), dim3(BS), 0, s>>>(x, w, mean, rstd, g, dx, part, rows, h);
  }
#undef OXI_BWD
}

// Bytes of column partials the backward needs for (rows, H): 2 x blocks x H
// floats, or 0 when neither dw nor db is wanted.
size_t bwd_part_bytes(bool need_part, int64_t rows, int64_t H, int cfg) {
  if (!need_part) return 0;
  const int tpr = cfg ? cfg / 10 : BS;
  const int nt = tpr == 64 ? (cfg % 10 <= 3 ? 1024 : 512) : tpr;  // bwd_threads<TPR, NV>()
  int64_t nblk = ceil_div(rows, nt / tpr);
  const int64_t cap = (int64_t)cu_count() * (nt == 1024 ? 1 : 2);
  if (nblk > cap) nblk = cap;
  if (nblk < 1) nblk = 1;
  return sizeof(float) * 2 * (size_t)nblk * (size_t)H;
}

// `fixed` (when not null) holds at least bwd_part_bytes() bytes of device
// memory for the column partials; otherwise they come from the caching
// allocator.
template <bool LN, int MODE, int ACT = ACT_NONE>
int launch_bwd(const float* x, const float* w, const float* b, const float* mean, const float* rstd,
               const float* g, float* dyo, float* dx, float* dw, float* db, int64_t rows, int64_t H,
               void* fixed = nullptr) {
  hipStream_t s = stream();
  const bool need_part = dw || (LN && db);
  const int cfg = vec_ok(H, {x, w, b, g, dyo, dx}) ? pick_bwd_cfg(H / 4) : 0;
  if (ACT != ACT_NONE && cfg == 0) return fail(OXI_OTHER, "norm_act_bwd: internal: unvectorized fused launch");
  const int tpr = cfg ? cfg / 10 : BS;
  const int nt = tpr == 64 ? (cfg % 10 <= 3 ? 1024 : 512) : tpr;  // bwd_threads<TPR, NV>()
  const int gpb = nt / tpr;
  // Blocks: enough to fill the chip, few enough that the partial rows stay
  // a small fraction of the row traffic.
  int64_t nblk = ceil_div(rows, gpb);
  // (measured: 2 blocks per CU beat 3 and 4 for 4096-float rows)
  const int64_t cap = (int64_t)cu_count() * (nt == 1024 ? 1 : 2);
  if (need_part && nblk > cap) nblk = cap;
  if (!need_part && nblk > (int64_t)cu_count() * 16) nblk = (int64_t)cu_count() * 16;
  if (nblk < 1) nblk = 1;
  Workspace ws(need_part && !fixed ? sizeof(float) * 2 * (size_t)nblk * (size_t)H : 0);
  if (need_part && !fixed && !ws.p) return OXI_OTHER;
  // no partials without dw/db: the kernel then writes none (its launch shape
  // may have more blocks than bwd_part_bytes() sizes for)
  float* part = !need_part ? nullptr : fixed ? static_cast<float*>(fixed) : ws.as<float>();
  const int h = (int)H;
  if (nt_stores(rows * H * 4))
    launch_bwd_cfg<LN, MODE, true, ACT>(cfg, s, nblk, nt, x, w, b, mean, rstd, g, dyo, dx, part, rows, h);
  else
    launch_bwd_cfg<LN, MODE, false, ACT>(cfg, s, nblk, nt, x, w, b, mean, rstd, g, dyo, dx, part, rows, h);
  int rc = check_launch(LN ? "layer_norm_bwd" : "rms_norm_bwd");
  if (rc != OXI_OK) return rc;
  if (need_part) {
    col_finish_k<<<dim3((unsigned)ceil_div(H, 64), LN ? 2 : 1), dim3(64 * FIN_W), 0, s>>>(part, (int)nblk, h, dw,
                                                                                    LN ? db : nullptr);
    rc = check_launch("norm_param_grad_finish");
  }
  return rc;
}

template <bool LN, int MODE>
int launch_act_bwd(int act, const float* x, const float* w, const float* b, const float* mean, const float* rstd,
                   const float* g, float* dyo, float* dx, float* dw, float* db, int64_t rows, int64_t H) {
  switch (act) {
    case OXI_ACT_GELU_TANH:
      return launch_bwd<LN, MODE, OXI_ACT_GELU_TANH>(x, w, b, mean, rstd, g, dyo, dx, dw, db, rows, H);
    case OXI_ACT_GELU_ERF:
      return launch_bwd<LN, MODE, OXI_ACT_GELU_ERF>(x, w, b, mean, rstd, g, dyo, dx, dw, db, rows, H);
    case OXI_ACT_SILU:
      return launch_bwd<LN, MODE, OXI_ACT_SILU>(x, w, b, mean, rstd, g, dyo, dx, dw, db, rows, H);
    case OXI_ACT_SOFTMAX:
      return launch_bwd<LN, MODE, OXI_ACT_SOFTMAX>(x, w, b, mean, rstd, g, dyo, dx, dw, db, rows, H);
    default:
      return launch_bwd<LN, MODE, OXI_ACT_LOG_SOFTMAX>(x, w, b, mean, rstd, g, dyo, dx, dw, db, rows, H);
  }
}

// Shared checks of the fused entry points; OXI_OK means "launch".
int check_act(const char* what, int act, int mode, const float* x, const float* w, const float* b, const float* g,
              const float* dyo, const float* dx, int64_t rows, int64_t cols) {
  if (act < OXI_ACT_GELU_TANH || act > OXI_ACT_LOG_SOFTMAX)
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
  return mode == OXI_NORM_VJP_REF
             ? launch_bwd<false, OXI_NORM_VJP_REF>(x, w, nullptr, nullptr, rstd, g, nullptr, dx, dw, nullptr, rows, cols)
             : launch_bwd<false, OXI_NORM_VJP_EXACT>(x, w, nullptr, nullptr, rstd, g, nullptr, dx, dw, nullptr, rows,
                                                     cols);
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
             ? launch_bwd<true, OXI_NORM_VJP_REF>(x, w, nullptr, mean, rstd, g, nullptr, dx, dw, db, rows, cols)
             : launch_bwd<true, OXI_NORM_VJP_EXACT>(x, w, nullptr, mean, rstd, g, nullptr, dx, dw, db, rows, cols);
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
  return mode == OXI_NORM_VJP_REF
             ? launch_bwd<true, OXI_NORM_VJP_REF>(x, w, nullptr, mean, rstd, g, nullptr, dx, dw, db, rows, cols, sp)
             : launch_bwd<true, OXI_NORM_VJP_EXACT>(x, w, nullptr, mean, rstd, g, nullptr, dx, dw, db, rows, cols,
                                                    sp);
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
  return mode == OXI_NORM_VJP_REF
             ? launch_act_bwd<false, OXI_NORM_VJP_REF>(act, x, w, nullptr, nullptr, rstd, g, dy, dx, dw, nullptr,
                                                       rows, cols)
             : launch_act_bwd<false, OXI_NORM_VJP_EXACT>(act, x, w, nullptr, nullptr, rstd, g, dy, dx, dw, nullptr,
                                                         rows, cols);
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
  return mode == OXI_NORM_VJP_REF
             ? launch_act_bwd<true, OXI_NORM_VJP_REF>(act, x, w, b, mean, rstd, g, dy, dx, dw, db, rows, cols)
             : launch_act_bwd<true, OXI_NORM_VJP_EXACT>(act, x, w, b, mean, rstd, g, dy, dx, dw, db, rows, cols);
}

}  // extern "C"
