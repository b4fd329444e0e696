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
// wider rows 1 per block. The leading-sum walk (LSUM) runs 4 waves to a
// block, each with LSUM_DEPTH rows in flight.
// The softmax positional-sum split's block (waves per position) and whether
// it loads x and g non-temporally. Measured at C5's (16, 1024, 768): 256
// threads with plain loads 40.7 us; non-temporal loads 47.1 us; 512 and
// 1024 threads (non-temporal) 47.4 and 52.0 us.
#ifndef OXI_LSUM_SPLIT_THREADS
#define OXI_LSUM_SPLIT_THREADS 256
#endif
#ifndef OXI_LSUM_SPLIT_NT
#define OXI_LSUM_SPLIT_NT 0
#endif
constexpr int LSUM_SPLIT_THREADS = OXI_LSUM_SPLIT_THREADS;  // a position's waves with a softmax
template <int TPR, int NV, bool LSUM = false, int ACT = OXI_ACT_NONE>
constexpr int bwd_threads() {
  return LSUM ? ((ACT == OXI_ACT_SOFTMAX || ACT == OXI_ACT_LOG_SOFTMAX) ? LSUM_SPLIT_THREADS : 256)
              : TPR == 64 ? (NV <= 3 ? 1024 : 512) : TPR;
}
constexpr int LSUM_THREADS = 256;
#ifndef OXI_LSUM_DEPTH
#define OXI_LSUM_DEPTH 4
#endif
constexpr int LSUM_DEPTH = OXI_LSUM_DEPTH;
// The softmax positional-sum split stages a position's dx rows (lead x H
// floats) in dynamic LDS when they take at most LSUM_STAGE_MAX bytes (one
// block within 64 KB of LDS with its static arrays); larger positions are
// re-read from dx.
#ifndef OXI_LSUM_STAGE_MAX
#define OXI_LSUM_STAGE_MAX (56 << 10)
#endif
__host__ __device__ constexpr bool lsum_staged(int64_t lead, int64_t H) {
  return lead * H * 4 <= OXI_LSUM_STAGE_MAX;
}

// ACT_NONE: g is the norm output's gradient. Otherwise g is the gradient of
// act(y) and the kernel first forms dy (written to dyo if set): g * act'(y)
// for the elementwise activations, the softmax VJP over the row for
// OXI_ACT_SOFTMAX / OXI_ACT_LOG_SOFTMAX.
constexpr int ACT_NONE = OXI_ACT_NONE;
constexpr bool is_softmax_act(int act) { return act == OXI_ACT_SOFTMAX || act == OXI_ACT_LOG_SOFTMAX; }

template <int ACT>
__device__ __forceinline__ float act_vjp(float y, float g) {
  if constexpr (ACT == OXI_ACT_GELU_TANH) return GeluTanhBwd{}(y, g);
  else if constexpr (ACT == OXI_ACT_GELU_ERF) return GeluErfBwd{}(y, g);
  else return SiluBwd{}(y, g);
}

// Waves per SIMD the register budget must allow: the softmax positional-sum
// split runs 4 blocks of 4 waves to a CU (at most 128 VGPRs); otherwise no
// bound beyond the block size.
template <bool LSUM, int ACT>
constexpr int bwd_waves_per_eu() { return LSUM && is_softmax_act(ACT) ? 4 : 1; }

template <int TPR, int NV, int MODE, bool LN, bool NTS, int ACT, bool LSUM>
__global__ __launch_bounds__((bwd_threads<TPR, NV, LSUM, ACT>())) __attribute__((amdgpu_waves_per_eu(bwd_waves_per_eu<LSUM, ACT>())))
void norm_bwd_k(const float* __restrict__ x, const float* __restrict__ w,
                                                 const float* __restrict__ b,
                                                 const float* __restrict__ mean, const float* __restrict__ rstd,
                                                 const float* __restrict__ g, float* __restrict__ dyo,
                                                 float* __restrict__ dx,
                                                 float* __restrict__ part, int64_t rows, int H,
                                                 float* __restrict__ lsum, int64_t T) {
  static_assert(!LSUM || TPR == 64, "the leading-sum walk takes one-wave rows");
  constexpr int NT = bwd_threads<TPR, NV, LSUM, ACT>();
  constexpr int GPB = NT / TPR;
  constexpr int ROWF = TPR * NV * 4;  // floats a group covers
  constexpr bool SPLIT = LSUM && is_softmax_act(ACT);
  __shared__ float lds[2 * (NT / 64)];
  // the softmax positional-sum split combines its groups in the dynamic LDS
  // (lsum_dyn_bytes), which first stages each position's dx rows
  __shared__ float comb_static[(GPB > 1 && !SPLIT) ? GPB * ROWF : 1];
  extern __shared__ __align__(16) float dyn_lds[];
  float* comb = SPLIT ? dyn_lds : comb_static;
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

  // The loop-invariant weights (and, for the activation prologue, biases)
  // never load inside the row loop: such a load is younger than the next
  // row's prefetch, and the in-order vmcnt wait for it would also wait for
  // the prefetch. Wide rows (TPR > 64) keep them in registers; one-wave rows
  // run 16 waves to a CU at up to 128 VGPRs and read them from LDS, staged
  // once per block. Padding lanes (c >= h4) are zeroed at use.
  constexpr bool REG_W = TPR > 64;
  constexpr int WL = REG_W ? 1 : TPR * NV;  // float4s of w (and b) in LDS
  __shared__ f4 wl[WL], bl[WL];
  f4 wr[NV], br[NV];
  const bool need_b = ACT != ACT_NONE && LN && b;
  if constexpr (REG_W) {
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int cc = min(k * TPR + t, h4 - 1);
      wr[k] = w ? w4[cc] : f4{1.f, 1.f, 1.f, 1.f};
      br[k] = need_b ? b4[cc] : zero;
    }
  } else {
    for (int c = threadIdx.x; c < WL; c += NT) {
      const int cc = min(c, h4 - 1);
      wl[c] = w ? w4[cc] : f4{1.f, 1.f, 1.f, 1.f};
      bl[c] = need_b ? b4[cc] : zero;
    }
    __syncthreads();
  }
  auto w_at = [&](int k) -> f4 {  // w's float4 k of this lane (in range lanes)
    if constexpr (REG_W) return wr[k];
    else return wl[k * TPR + t];
  };
  auto b_at = [&](int k) -> f4 {
    if constexpr (REG_W) return br[k];
    else return bl[k * TPR + t];
  };
  auto wv_at = [&](int k) -> f4 { return k * TPR + t < h4 ? w_at(k) : zero; };

  // Rows are double-buffered: the next row's x, g and statistics are in
  // flight while the current row is reduced and stored. The two register
  // sets swap roles every row (the loop is unrolled twice, so no copies: a
  // copy of a loading register waits for its load) and every prefetch load
  // issues (row and column clamped in bounds), so the wait before a row's
  // first use counts exactly the younger loads.
  const int64_t ngroups = (int64_t)gridDim.x * GPB;
  int64_t row = (int64_t)blockIdx.x * GPB + gi;
  int red = 0;  // reductions so far: consecutive ones use alternate LDS slot sets
  auto slot = [&]() { return lds + ((red++ & 1) ? NT / 64 : 0); };
  auto fetch = [&](RowTile<TPR, NV>& xt, RowTile<TPR, NV>& gt, float& inv, float& mu, int64_t r) {
    r = r < rows ? r : rows - 1;
    // the lead-sum walk's last refills re-read a row it has just read: plain
    // loads keep it in L2 (non-temporal ones fetched it from HBM again, +25%
    // reads at 16 rows a position)
    constexpr bool ntl = !LSUM || (is_softmax_act(ACT) && OXI_LSUM_SPLIT_NT);
    xt.template load_clamped<ntl>(x + r * H, h4, t);
    gt.template load_clamped<ntl>(g + r * H, h4, t);
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
          if (w) yv = yv * w_at(k);
          if (LN && b) yv = yv + b_at(k);
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
          if (w) yv = yv * w_at(k);
          if (LN && b) yv = yv + b_at(k);
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
  // The scheduling barriers keep the current row's first use below the next
  // row's loads, so its wait leaves those loads in flight.
  if constexpr (LSUM && is_softmax_act(ACT)) {
    // Rows are (lead, T): row b * T + p is batch b at position p. The softmax
    // prologue makes a row's VJP long, so a position's rows are spread over
    // the block's waves rather than walked by one: a block owns positions
    // p = block, block + blocks, ...; for each, wave gi forms the VJP of its
    // contiguous share of the batch rows (each row reduced within one wave,
    // as the node-by-node kernels do, so dx has their bits) and writes dx.
    // After a barrier the block's threads take the row's columns, and each
    // adds its column over the position's rows in batch order, starting from
    // 0.0f: the sequential sum oxi_reduce(SUM) forms over the leading dim,
    // bit for bit. The rows come from LDS, where each wave also put its dx
    // rows, when the position fits there (lsum_staged; 48 KB at C5), else
    // from dx again. One wave per position walking all its rows (below) runs
    // this VJP at one wave per SIMD: 42-44 us at C5's (16, 1024, 768);
    // split, re-reading dx through the caches (the x and g streams evict
    // most of it from L2: 38% more HBM fetch than the pass needs): 39-41 us;
    // staged in LDS: 36.6-36.9 us against 39.4 in the same runs; the pass
    // without the positional sum: 33 us.
    const int lead = (int)(rows / T);
    const int q = (lead + GPB - 1) / GPB;  // rows of a position per wave
    const int b0 = gi * q;
    const int nb = max(0, min(lead, b0 + q) - b0);
    // a position's dx rows fit the dynamic LDS: the column sums read them
    // there (the same values, added in the same order)
    const bool staged = lsum_staged(lead, H);
    f4* const stage = reinterpret_cast<f4*>(dyn_lds);
    auto stage_row = [&](const RowTile<TPR, NV>& dt, int bb) {
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        const int c = k * TPR + t;
        if (c < h4) stage[(int64_t)bb * h4 + c] = dt.v[k];
      }
    };
    for (int64_t p = blockIdx.x; p < T; p += gridDim.x) {
      if (nb > 0) {
        // two rows in flight; every prefetch issues (past the wave's last row
        // it re-reads that row), so each wait counts exactly the younger loads
        const int64_t r_first = (int64_t)b0 * T + p;
        auto rj = [&](int j) { return r_first + (int64_t)min(j, nb - 1) * T; };
        fetch(xa, ga, ia, ma, rj(0));
        for (int j = 0; j < nb; j += 2) {
          fetch(xb, gb, ib, mb, rj(j + 1));
          __builtin_amdgcn_sched_barrier(0);
          process(xa, ga, ia, ma, rj(j));  // ga now holds the row's dx
          if (staged) stage_row(ga, b0 + j);
          if (j + 1 >= nb) break;
          fetch(xa, ga, ia, ma, rj(j + 2));
          __builtin_amdgcn_sched_barrier(0);
          process(xb, gb, ib, mb, rj(j + 1));
          if (staged) stage_row(gb, b0 + j + 1);
        }
      }
      __syncthreads();  // every dx row of position p is written (and staged)
      if (staged) {
        for (int c = threadIdx.x; c < h4; c += NT) {
          const f4* src = stage + c;
          f4 acc = zero;
          for (int bb = 0; bb < lead; ++bb) acc = acc + src[(int64_t)bb * h4];
          st_stream<NTS>(acc, reinterpret_cast<f4*>(lsum + p * H) + c);
        }
        __syncthreads();  // the next position's rows overwrite the stage
      } else {
        for (int c = threadIdx.x; c < h4; c += NT) {
          const f4* src = reinterpret_cast<const f4*>(dx + p * H) + c;
          const int64_t step = T * (int64_t)h4;  // float4s from one batch row to the next
          f4 acc = zero;
          int bb = 0;
          for (; bb + 4 <= lead; bb += 4) {
            const f4 v0 = src[(int64_t)bb * step], v1 = src[(int64_t)(bb + 1) * step];
            const f4 v2 = src[(int64_t)(bb + 2) * step], v3 = src[(int64_t)(bb + 3) * step];
            acc = acc + v0;
            acc = acc + v1;
            acc = acc + v2;
            acc = acc + v3;
          }
          for (; bb < lead; ++bb) acc = acc + src[(int64_t)bb * step];
          st_stream<NTS>(acc, reinterpret_cast<f4*>(lsum + p * H) + c);
        }
      }
    }
  } else if constexpr (LSUM) {
    // Rows are (lead, T): row b * T + p is batch b at position p. Each wave
    // owns positions p = wave, wave + waves, ... and walks a position's rows
    // in batch order, LSUM_DEPTH rows in flight (the row sequence continues
    // into the wave's next position), adding each dx row to a register sum
    // that starts from 0.0f: the sequential sum oxi_reduce(SUM) forms over
    // the leading dim, bit for bit. No barriers. lead is a multiple of
    // LSUM_DEPTH (the host checks), so every round processes LSUM_DEPTH rows
    // and every refill load issues: the waits count exactly the younger
    // loads. The last round's refills re-read the wave's last row (from L2).
    const int lead = (int)(rows / T);
    const int waves = (int)gridDim.x * GPB;
    const int wave = (int)blockIdx.x * GPB + gi;
    const int npos = wave < T ? (int)((T - 1 - wave) / waves + 1) : 0;
    const int nj = npos * lead;  // this wave's rows
    const int last_p = wave + (npos - 1) * waves;
    int fb = 0, fp = wave;  // the next row to fetch: batch fb at position fp
    int cb = 0, cp = wave;  // the next row to process
    auto fetch_next = [&](RowTile<TPR, NV>& xt, RowTile<TPR, NV>& gt, float& inv, float& mu) {
      const int64_t r = fp <= last_p ? (int64_t)fb * T + fp : (int64_t)(lead - 1) * T + last_p;
      fetch(xt, gt, inv, mu, r);
      if (++fb == lead) {
        fb = 0;
        fp += waves;
      }
    };
    if (nj > 0) {
      RowTile<TPR, NV> xs[LSUM_DEPTH], gs[LSUM_DEPTH];
      float is[LSUM_DEPTH], ms[LSUM_DEPTH];
      f4 acc[NV];
#pragma unroll
      for (int d = 0; d < LSUM_DEPTH; ++d) fetch_next(xs[d], gs[d], is[d], ms[d]);
      for (int j0 = 0; j0 < nj; j0 += LSUM_DEPTH) {
#pragma unroll
        for (int d = 0; d < LSUM_DEPTH; ++d) {
          process(xs[d], gs[d], is[d], ms[d], (int64_t)cb * T + cp);  // gs[d] now holds the row's dx
          if (cb == 0) {
#pragma unroll
            for (int q = 0; q < NV; ++q) acc[q] = zero;
          }
#pragma unroll
          for (int q = 0; q < NV; ++q) acc[q] = acc[q] + gs[d].v[q];
          if (cb == lead - 1) {
            f4* o = reinterpret_cast<f4*>(lsum + (int64_t)cp * H);
#pragma unroll
            for (int q = 0; q < NV; ++q)
              if (q * TPR + t < h4) st_stream<NTS>(acc[q], o + q * TPR + t);
          }
          if (++cb == lead) {
            cb = 0;
            cp += waves;
          }
          // the refill reuses the slot's registers after their last use
          __builtin_amdgcn_sched_barrier(0);
          fetch_next(xs[d], gs[d], is[d], ms[d]);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
  } else if ((int64_t)rows <= ngroups) {
    // at most one row per group (e.g. 4096 rows of 768): nothing to prefetch
    if (row < rows) {
      fetch(xa, ga, ia, ma, row);
      process(xa, ga, ia, ma, row);
    }
  } else {
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

// Dynamic LDS of a lead-sum launch: for the softmax split, its group combine
// (4 groups x 64 lanes x NV float4s) or, when staged, the position's dx rows
// if larger; nothing for the walk.
template <int NV, int ACT>
size_t lsum_dyn_bytes(int64_t lead, int64_t H) {
  if (!is_softmax_act(ACT)) return 0;
  const size_t comb = sizeof(float) * (size_t)(LSUM_SPLIT_THREADS / 64) * (64 * NV * 4);
  const size_t stage = lsum_staged(lead, H) ? sizeof(float) * (size_t)(lead * H) : 0;
  return std::max(comb, stage);
}

template <bool LN, int MODE, bool NTS, int ACT>
void launch_bwd_cfg(int cfg, hipStream_t s, int64_t nblk, int nt, const float* x, const float* w, const float* b,
                    const float* mean, const float* rstd, const float* g, float* dyo, float* dx, float* part,
                    int64_t rows, int h, float* lsum, int64_t T) {
#define OXI_BWD(TPR, NV)                                                                                   \
  case TPR * 10 + NV:                                                                                      \
    norm_bwd_k<TPR, NV, MODE, LN, NTS, ACT, false><<<dim3((unsigned)nblk), dim3(nt), 0, s>>>(              \
        x, w, b, mean, rstd, g, dyo, dx, part, rows, h, nullptr, 0);                                       \
    break;
#define OXI_BWD_LSUM(NV)                                                                                   \
  case 640 + NV:                                                                                           \
    norm_bwd_k<64, NV, MODE, LN, NTS, ACT, true><<<dim3((unsigned)nblk), dim3(bwd_threads<64, NV, true, ACT>()), \
                                                   lsum_dyn_bytes<NV, ACT>(rows / T, h), s>>>(              \
        x, w, b, mean, rstd, g, dyo, dx, part, rows, h, lsum, T);                                          \
    break;
  if (lsum) {  // one-wave rows only (lsum_check)
    switch (cfg) {
      OXI_BWD_LSUM(1)
      OXI_BWD_LSUM(2)
      OXI_BWD_LSUM(3)
      OXI_BWD_LSUM(4)
      default:
        break;
    }
    return;
  }
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
#undef OXI_BWD_LSUM
}

// 1024-thread (one-wave row) blocks per CU: 2 made C5's layer_norm + silu
// VJP 43 us against 35 us at 1 (C1's rms_norm VJP unchanged)
#ifndef OXI_BWD_BPC1024
#define OXI_BWD_BPC1024 1
#endif
// Blocks per CU of a backward launch of nt-thread blocks that writes column
// partials (the softmax positional-sum split aside); the partial buffer's
// size and the launch both come from it. (measured: 2 blocks per CU beat 3
// and 4 for 4096-float rows)
constexpr int bwd_blocks_per_cu(int nt) { return nt == 1024 ? OXI_BWD_BPC1024 : 2; }

// Bytes of column partials the backward needs for (rows, H): 2 x blocks x H
// floats, or 0 when neither dw nor db is wanted.
size_t bwd_part_bytes(bool need_part, int64_t rows, int64_t H, int cfg) {
  if (!need_part) return 0;
  const int tpr = cfg ? cfg / 10 : BS;
  const int nt = tpr == 64 ? (cfg % 10 <= 3 ? 1024 : 512) : tpr;  // bwd_threads<TPR, NV>()
  int64_t nblk = ceil_div(rows, nt / tpr);
  const int64_t cap = (int64_t)cu_count() * bwd_blocks_per_cu(nt);
  if (nblk > cap) nblk = cap;
  if (nblk < 1) nblk = 1;
  return sizeof(float) * 2 * (size_t)nblk * (size_t)H;
}

// `fixed` (when not null) is fixed_bytes of device memory for the column
// partials, which must hold bwd_part_bytes() (checked before any launch);
// otherwise they come from the caching allocator.
// lsum (with lead > 0): also write lsum (rows / lead, H) = the sum of dx over
// the leading dim of a (lead, rows / lead) row grid; the caller has checked
// lsum_ok().
template <bool LN, int MODE, int ACT = ACT_NONE>
int launch_bwd(const float* x, const float* w, const float* b, const float* mean, const float* rstd,
               const float* g, float* dyo, float* dx, float* dw, float* db, int64_t rows, int64_t H,
               void* fixed = nullptr, float* lsum = nullptr, int64_t lead = 0, size_t fixed_bytes = 0) {
  hipStream_t s = stream();
  const bool need_part = dw || (LN && db);
  const int cfg = vec_ok(H, {x, w, b, g, dyo, dx}) ? pick_bwd_cfg(H / 4) : 0;
  if (ACT != ACT_NONE && cfg == 0) return fail(OXI_OTHER, "norm_act_bwd: internal: unvectorized fused launch");
  const int tpr = cfg ? cfg / 10 : BS;
  const bool split = lsum && is_softmax_act(ACT);
  const int nt = lsum ? (split ? LSUM_SPLIT_THREADS : LSUM_THREADS) : tpr == 64 ? (cfg % 10 <= 3 ? 1024 : 512) : tpr;  // bwd_threads<>()
  const int gpb = nt / tpr;
  // Blocks: enough to fill the chip, few enough that the partial rows stay
  // a small fraction of the row traffic.
  // lsum: a wave per position, or with a softmax a block per position
  int64_t nblk = lsum ? (split ? rows / lead : ceil_div(rows / lead, gpb)) : ceil_div(rows, gpb);
  // blocks per CU of the split (2, 3, 4 at C5: 40.4, 40.1, 40.2 us)
#ifndef OXI_LSUM_SPLIT_BPC
#define OXI_LSUM_SPLIT_BPC (1024 / LSUM_SPLIT_THREADS)
#endif
  const int64_t cap = (int64_t)cu_count() * (split ? OXI_LSUM_SPLIT_BPC : bwd_blocks_per_cu(nt));
  if (need_part && nblk > cap) nblk = cap;
  if (!need_part && nblk > (int64_t)cu_count() * 16) nblk = (int64_t)cu_count() * 16;
  if (nblk < 1) nblk = 1;
  const size_t part_bytes = need_part ? sizeof(float) * 2 * (size_t)nblk * (size_t)H : 0;
  if (fixed && part_bytes > fixed_bytes)
    return fail(OXI_OTHER, "norm VJP: internal: column partials of %zu bytes exceed the fixed buffer of %zu bytes",
                part_bytes, fixed_bytes);
  Workspace ws(!fixed ? part_bytes : 0);
  if (need_part && !fixed && !ws.p) return fail_alloc("norm VJP: column partials");
  // no partials without dw/db: the kernel then writes none (its launch shape
  // may have more blocks than bwd_part_bytes() sizes for)
  float* part = !need_part ? nullptr : fixed ? static_cast<float*>(fixed) : ws.as<float>();
  const int h = (int)H;
  const int64_t T = lsum ? rows / lead : 0;
  if (nt_stores(rows * H * 4))
    launch_bwd_cfg<LN, MODE, true, ACT>(cfg, s, nblk, nt, x, w, b, mean, rstd, g, dyo, dx, part, rows, h, lsum, T);
  else
    launch_bwd_cfg<LN, MODE, false, ACT>(cfg, s, nblk, nt, x, w, b, mean, rstd, g, dyo, dx, part, rows, h, lsum, T);
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
                   const float* g, float* dyo, float* dx, float* dw, float* db, int64_t rows, int64_t H,
                   float* lsum = nullptr, int64_t lead = 0) {
  switch (act) {
    case OXI_ACT_NONE:
      return launch_bwd<LN, MODE>(x, w, b, mean, rstd, g, nullptr, dx, dw, db, rows, H, nullptr, lsum, lead);
    case OXI_ACT_GELU_TANH:
      return launch_bwd<LN, MODE, OXI_ACT_GELU_TANH>(x, w, b, mean, rstd, g, dyo, dx, dw, db, rows, H, nullptr,
                                                     lsum, lead);
    case OXI_ACT_GELU_ERF:
      return launch_bwd<LN, MODE, OXI_ACT_GELU_ERF>(x, w, b, mean, rstd, g, dyo, dx, dw, db, rows, H, nullptr, lsum,
                                                    lead);
    case OXI_ACT_SILU:
      return launch_bwd<LN, MODE, OXI_ACT_SILU>(x, w, b, mean, rstd, g, dyo, dx, dw, db, rows, H, nullptr, lsum,
                                                lead);
    case OXI_ACT_SOFTMAX:
      return launch_bwd<LN, MODE, OXI_ACT_SOFTMAX>(x, w, b, mean, rstd, g, dyo, dx, dw, db, rows, H, nullptr, lsum,
                                                   lead);
    default:
      return launch_bwd<LN, MODE, OXI_ACT_LOG_SOFTMAX>(x, w, b, mean, rstd, g, dyo, dx, dw, db, rows, H, nullptr,
                                                       lsum, lead);
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
             ? launch_bwd<true, OXI_NORM_VJP_REF>(x, w, nullptr, mean, rstd, g, nullptr, dx, dw, db, rows, cols, sp,
                                                  nullptr, 0, (size_t)OXI_NOALLOC_SCRATCH_BYTES)
             : launch_bwd<true, OXI_NORM_VJP_EXACT>(x, w, nullptr, mean, rstd, g, nullptr, dx, dw, db, rows, cols,
                                                    sp, nullptr, 0, (size_t)OXI_NOALLOC_SCRATCH_BYTES);
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
  return mode == OXI_NORM_VJP_REF
             ? launch_act_bwd<false, OXI_NORM_VJP_REF>(act, x, w, nullptr, nullptr, rstd, g, dy, dx, dw, nullptr,
                                                       rows, cols, dx_sum, lead)
             : launch_act_bwd<false, OXI_NORM_VJP_EXACT>(act, x, w, nullptr, nullptr, rstd, g, dy, dx, dw, nullptr,
                                                         rows, cols, dx_sum, lead);
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
  return mode == OXI_NORM_VJP_REF
             ? launch_act_bwd<true, OXI_NORM_VJP_REF>(act, x, w, b, mean, rstd, g, dy, dx, dw, db, rows, cols, dx_sum,
                                                      lead)
             : launch_act_bwd<true, OXI_NORM_VJP_EXACT>(act, x, w, b, mean, rstd, g, dy, dx, dw, db, rows, cols,
                                                        dx_sum, lead);
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
