// The norm VJP kernels and their launch (see norm_bwd.h): included only by
// the translation units that instantiate them.
#pragma once

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
// Backward, register-resident rows, grid-strided over rows, column partials.
//
// part (if not null): [2][gridDim.x][H] floats, dw partials then db partials.

// Threads per backward block: one-wave rows run 16 to a block (one block per
// CU: 16 waves in flight, one partial row per CU), or 8 to a block (two
// blocks per CU) when 4 float4s per lane would not fit the registers of 16;
// wider rows 1 per block. The leading-sum walk (LSUM) runs 4 waves to a
// block, each with LSUM_DEPTH rows in flight.
// The softmax positional-sum split's block (waves per position) and whether
// it loads x and g non-temporally. Measured at C5's (16, 1024, 768), in the
// warm step: since the dx rows are staged in LDS (nothing re-read through
// L2), non-temporal loads take 33-34 us against 44 us with plain ones, whose
// lines evict the next kernels' inputs. 512-thread blocks (8 rows a chunk,
// half the barriers) took 39.6-40.0 us in the step against 37.0-37.4 us.
// Earlier, with dx re-read from L2,
// 256 threads measured 40.7 us with plain loads and 47.1 us with
// non-temporal ones, 512 and 1024 threads 47.4 and 52.0 us.
#ifndef OXI_LSUM_SPLIT_THREADS
#define OXI_LSUM_SPLIT_THREADS 256
#endif
#ifndef OXI_LSUM_SPLIT_NT
#define OXI_LSUM_SPLIT_NT 1
#endif
constexpr int LSUM_SPLIT_THREADS = OXI_LSUM_SPLIT_THREADS;  // a position's waves with a softmax
template <int TPR, int NV, bool LSUM = false, int ACT = OXI_ACT_NONE>
constexpr int bwd_threads() {
  return LSUM ? ((ACT == OXI_ACT_SOFTMAX || ACT == OXI_ACT_LOG_SOFTMAX) ? LSUM_SPLIT_THREADS : 256)
              : TPR == 64 ? (NV <= 3 ? 1024 : 512) : TPR;
}
constexpr int LSUM_THREADS = 256;
// ACT_NONE: g is the norm output's gradient. Otherwise g is the gradient of
// act(y) and the kernel first forms dy (written to dyo if set): g * act'(y)
// for the elementwise activations, the softmax VJP over the row for
// OXI_ACT_SOFTMAX / OXI_ACT_LOG_SOFTMAX.
constexpr int ACT_NONE = OXI_ACT_NONE;

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

// FULL: rows of exactly TPR * NV float4s (H = 4 * TPR * NV), so that H and
// the float4 count are compile-time constants: no lane is padding, and the
// bounds checks, padding selects and row-address multiplies fold away (the
// per-row instruction count of C5's fused softmax VJP drops by a third).
template <int TPR, int NV, int MODE, bool LN, bool NTS, int ACT, bool LSUM, bool FULL>
__global__ __launch_bounds__((bwd_threads<TPR, NV, LSUM, ACT>())) __attribute__((amdgpu_waves_per_eu(bwd_waves_per_eu<LSUM, ACT>())))
void norm_bwd_k(const float* __restrict__ x, const float* __restrict__ w,
                                                 const float* __restrict__ b,
                                                 const float* __restrict__ mean, const float* __restrict__ rstd,
                                                 const float* __restrict__ g, float* __restrict__ dyo,
                                                 float* __restrict__ dx,
                                                 float* __restrict__ part, int64_t rows, int H_arg,
                                                 float* __restrict__ lsum, int64_t T) {
  const int H = FULL ? 4 * TPR * NV : H_arg;
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
        div_by_sum<NV>(pk, s);  // e / s, rounded as the division operator rounds it
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
    // the block's GPB waves: a block owns positions p = block, block +
    // blocks, ..., and walks each position's batch in chunks of GPB rows,
    // wave gi forming the VJP of row b = chunk * GPB + gi (each row reduced
    // within one wave, as the node-by-node kernels do, so dx has their bits),
    // writing dx and staging it in LDS. After a barrier the block's first h4
    // threads each add the chunk's staged rows, in batch order, to a running
    // sum of one float4 column kept in registers, which starts from 0.0f at
    // the position's first chunk: the sequential sum oxi_reduce(SUM) forms
    // over the leading dim, bit for bit. Each wave's next row (the next chunk
    // or position) is in flight across the barriers. Staging GPB rows rather
    // than the whole position keeps a block within GPB * H * 4 bytes of LDS
    // (12 KB at C5's 768 floats), so every position's block is resident at
    // once; staging all 16 rows (48 KB) held three blocks to a CU.
    static_assert(TPR * NV <= NT, "a column float4 per thread");
    const int lead = (int)(rows / T);
    const int nchunk = (lead + GPB - 1) / GPB;
    f4* const stage = reinterpret_cast<f4*>(dyn_lds);  // GPB rows of h4 float4s
    f4* const lsum4 = reinterpret_cast<f4*>(lsum);
    const int64_t npos = (int64_t)blockIdx.x < T ? (T - 1 - blockIdx.x) / gridDim.x + 1 : 0;
    const int64_t nk = npos * nchunk;  // (position, chunk) steps of this block
    // Two cursors over the block's steps (position p, chunk ck): the next row
    // to fetch and the next row to process. A step's row for this wave is
    // b = ck * GPB + gi; where the chunk has none (valid = false) the wave
    // fetches a row of the same position and never processes it; past the
    // last step it fetches the last position's row.
    int64_t p_f = blockIdx.x, p_p = blockIdx.x;
    int ck_f = 0, ck_p = 0;
    auto next_fetch = [&](bool& valid) -> int64_t {
      const int bb = ck_f * GPB + gi;
      valid = bb < lead;
      const int64_t r = (int64_t)min(bb, lead - 1) * T + min(p_f, T - 1);
      if (++ck_f == nchunk) {
        ck_f = 0;
        p_f += gridDim.x;
      }
      return r;
    };
    f4 acc = zero;
    auto chunk_step = [&](RowTile<TPR, NV>& xt, RowTile<TPR, NV>& gt, const float inv, const float mu,
                          const int64_t r, const bool valid) {
      if (valid) {
        process(xt, gt, inv, mu, r);  // gt now holds the row's dx
#pragma unroll
        for (int kk = 0; kk < NV; ++kk) {
          const int c = kk * TPR + t;
          if (c < h4) stage[gi * h4 + c] = gt.v[kk];
        }
      }
      __syncthreads();  // the chunk's dx rows are staged
      const int n = min(GPB, lead - ck_p * GPB);
      if ((int)threadIdx.x < h4) {
        if (ck_p == 0) acc = zero;
        for (int j = 0; j < n; ++j) acc = acc + stage[j * h4 + threadIdx.x];
        if (ck_p == nchunk - 1) st_stream<NTS>(acc, lsum4 + p_p * h4 + threadIdx.x);
      }
      if (++ck_p == nchunk) {
        ck_p = 0;
        p_p += gridDim.x;
      }
      __syncthreads();  // the next chunk's rows overwrite the stage
    };
    if (nk > 0) {
      bool va = false, vb = false;
      int64_t ra = next_fetch(va), rb = 0;
      fetch(xa, ga, ia, ma, ra);
      for (int64_t k = 0; k < nk; k += 2) {
        rb = next_fetch(vb);
        fetch(xb, gb, ib, mb, rb);
        __builtin_amdgcn_sched_barrier(0);
        chunk_step(xa, ga, ia, ma, ra, va);
        if (k + 1 >= nk) break;
        ra = next_fetch(va);
        fetch(xa, ga, ia, ma, ra);
        __builtin_amdgcn_sched_barrier(0);
        chunk_step(xb, gb, ib, mb, rb, vb);
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
// A block owns FIN_C columns; its threads form FS slices of FIN_C lanes,
// slice s summing the rows b = s, s + FS, ... (FIN_U loads in flight: up to
// FS * FIN_U partial rows in one round), then eight threads per column add
// the slice sums in slice order in two steps. blockIdx.y selects the dw (0)
// or db (1) plane. FS = 16 (256-thread blocks) when the partial rows fit one
// round, else 64: C1's rms_norm VJP (256 partial rows) 11.7-11.8 us in the
// step against 12.2 at 64 slices; C5's positional-sum VJP (1024 partial
// rows) 38.3-38.5 us at 64 slices against 39.0-39.1 at 16. Earlier, 64
// columns x 16 slices per block took 5.6-6.7 us at C5.
constexpr int FIN_C = 16;
constexpr int FIN_U = 16;

template <int FS>
__global__ __launch_bounds__(FIN_C * FS) void col_finish_k(const float* __restrict__ part, int nb, int H,
                                                         float* __restrict__ out0, float* __restrict__ out1) {
  constexpr int FIN_S = FS;
  float* out = blockIdx.y ? out1 : out0;
  if (!out) return;
  const float* p = part + (int64_t)blockIdx.y * nb * H;
  const int lane = threadIdx.x % FIN_C;
  const int slice = threadIdx.x / FIN_C;
  const int c = blockIdx.x * FIN_C + lane;
  const int cc = min(c, H - 1);  // in range: loads issue together
  double acc = 0.0;
  for (int b0 = slice; b0 < nb; b0 += FIN_S * FIN_U) {
    float v[FIN_U];
#pragma unroll
    for (int q = 0; q < FIN_U; ++q) v[q] = p[(int64_t)min(b0 + FIN_S * q, nb - 1) * H + cc];
#pragma unroll
    for (int q = 0; q < FIN_U; ++q)
      if (b0 + FIN_S * q < nb) acc += (double)v[q];
  }
  __shared__ double s[FIN_S][FIN_C];
  __shared__ double s8[8][FIN_C];
  s[slice][lane] = acc;
  __syncthreads();
  if (slice < 8) {
    double t = s[slice * (FIN_S / 8)][lane];
#pragma unroll
    for (int i = 1; i < FIN_S / 8; ++i) t += s[slice * (FIN_S / 8) + i][lane];
    s8[slice][lane] = t;
  }
  __syncthreads();
  if (slice == 0 && c < H) {
    double t = s8[0][lane];
#pragma unroll
    for (int i = 1; i < 8; ++i) t += s8[i][lane];
    out[c] = (float)t;
  }
}

// Dynamic LDS of a lead-sum launch: for the softmax split, its group combine
// (GPB groups x 64 lanes x NV float4s), which also holds a chunk's staged dx
// rows (GPB rows of at most 64 x NV float4s); nothing for the walk.
template <int NV, int ACT>
size_t lsum_dyn_bytes() {
  if (!is_softmax_act(ACT)) return 0;
  return sizeof(float) * (size_t)(LSUM_SPLIT_THREADS / 64) * (64 * NV * 4);
}

template <bool LN, int MODE, bool NTS, int ACT>
void launch_bwd_cfg(int cfg, hipStream_t s, int64_t nblk, int nt, const float* x, const float* w, const float* b,
                    const float* mean, const float* rstd, const float* g, float* dyo, float* dx, float* part,
                    int64_t rows, int h, float* lsum, int64_t T) {
#define OXI_BWD(TPR, NV)                                                                                   \
  case TPR * 10 + NV:                                                                                      \
    if (h == 4 * TPR * NV)                                                                                 \
      norm_bwd_k<TPR, NV, MODE, LN, NTS, ACT, false, true><<<dim3((unsigned)nblk), dim3(nt), 0, s>>>(      \
          x, w, b, mean, rstd, g, dyo, dx, part, rows, h, nullptr, 0);                                     \
    else                                                                                                   \
      norm_bwd_k<TPR, NV, MODE, LN, NTS, ACT, false, false><<<dim3((unsigned)nblk), dim3(nt), 0, s>>>(     \
          x, w, b, mean, rstd, g, dyo, dx, part, rows, h, nullptr, 0);                                     \
    break;
#define OXI_BWD_LSUM(NV)                                                                                   \
  case 640 + NV:                                                                                           \
    if (h == 4 * 64 * NV)                                                                                  \
      norm_bwd_k<64, NV, MODE, LN, NTS, ACT, true, true>                                                   \
          <<<dim3((unsigned)nblk), dim3(bwd_threads<64, NV, true, ACT>()), lsum_dyn_bytes<NV, ACT>(), s>>>( \
              x, w, b, mean, rstd, g, dyo, dx, part, rows, h, lsum, T);                                    \
    else                                                                                                   \
      norm_bwd_k<64, NV, MODE, LN, NTS, ACT, true, false>                                                  \
          <<<dim3((unsigned)nblk), dim3(bwd_threads<64, NV, true, ACT>()), lsum_dyn_bytes<NV, ACT>(), s>>>( \
              x, w, b, mean, rstd, g, dyo, dx, part, rows, h, lsum, T);                                    \
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
  // blocks per CU of the split: up to 32 waves to a CU, so one block per
  // position at C5's 1024 positions
#ifndef OXI_LSUM_SPLIT_BPC
#define OXI_LSUM_SPLIT_BPC (2048 / LSUM_SPLIT_THREADS)
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
    const dim3 fg((unsigned)ceil_div(H, FIN_C), LN ? 2 : 1);
    if (nblk <= 16 * FIN_U)
      col_finish_k<16><<<fg, dim3(FIN_C * 16), 0, s>>>(part, (int)nblk, h, dw, LN ? db : nullptr);
    else
      col_finish_k<64><<<fg, dim3(FIN_C * 64), 0, s>>>(part, (int)nblk, h, dw, LN ? db : nullptr);
    rc = check_launch("norm_param_grad_finish");
  }
  return rc;
}

// The launch for activation ACT in the four (norm, mode) combinations.
template <int ACT>
int norm_bwd_dispatch(bool ln, int mode, const NormBwdArgs& a) {
  const bool ref = mode == OXI_NORM_VJP_REF;
#define OXI_NB(LN, MODE)                                                                                   \
  launch_bwd<LN, MODE, ACT>(a.x, a.w, a.b, a.mean, a.rstd, a.g, a.dyo, a.dx, a.dw, a.db, a.rows, a.H, a.fixed, \
                            a.lsum, a.lead, a.fixed_bytes)
  if (ln) return ref ? OXI_NB(true, OXI_NORM_VJP_REF) : OXI_NB(true, OXI_NORM_VJP_EXACT);
  return ref ? OXI_NB(false, OXI_NORM_VJP_REF) : OXI_NB(false, OXI_NORM_VJP_EXACT);
#undef OXI_NB
}

}  // namespace
}  // namespace oxi
