// Softmax, log-softmax and fused cross-entropy kernels for gfx950.
//
// Softmax-family ops reduce over the middle dim of a contiguous
// (outer, len, inner) buffer. inner == 1 (the last dim, the hot case) runs one
// row per row group with the row held in registers when it fits
// (len <= 8192, 16-byte aligned), so x is read once and y written once;
// longer rows stream twice (online max/sum pass, then the write pass).
// inner > 1 runs one thread per (outer, inner) column, coalesced across inner.
//
// Cross-entropy (mean reduction) is fused into two kernels: the forward streams
// each logits row once with an online (max, sum-exp) and writes the row's
// log-sum-exp plus its picked log-probability; a one-block kernel forms the
// mean in float64 in fixed order. The backward streams logits once more and
// writes (softmax - onehot) * g / n. Bytes per row: 1 read fwd, 1 read + 1
// write bwd, instead of the reference's dense one-hot and ~16 passes
// (python/oxitorch/nn/functional.py:277-293).
#include <cmath>

#include "internal.h"
#include "rowtile.h"

namespace oxi {
namespace {

constexpr int BS = 256;

// Running (max, sum of exp(v - max)) of one thread; `m == -inf` means no
// finite contribution yet (sum 0).
struct Online {
  float m = NEG_INF;
  float s = 0.f;
  __device__ __forceinline__ void add4(const f4& v) {
    const float cm = max4(v);
    if (cm > m) {
      s = (m == NEG_INF) ? 0.f : s * expf(m - cm);
      m = cm;
    }
    if (m != NEG_INF) s += sum4(exp4(v - m));
    else if (cm != cm || v.x != v.x || v.y != v.y || v.z != v.z || v.w != v.w) s = __builtin_nanf("");
  }
  __device__ __forceinline__ void add1(float v) {
    if (v > m) {
      s = (m == NEG_INF) ? 0.f : s * expf(m - v);
      m = v;
    }
    if (m != NEG_INF) s += expf(v - m);
    else if (v != v) s = __builtin_nanf("");
  }
};

// Combine the Online states of a row group; every thread gets (M, S).
template <int TPR>
__device__ __forceinline__ void group_online(Online& o, float* lds) {
  const float M = group_max<TPR>(o.m, lds);
  float part = (o.m == NEG_INF) ? ((o.s != o.s) ? o.s : 0.f) : o.s * expf(o.m - M);
  const float S = group_sum<TPR, float>(part, lds + BS / 64);
  o.m = M;
  o.s = S;
}

// ---------------------------------------------------------------------------
// Last-dim kernels, register-resident rows.

template <int TPR, int NV, bool LOG, bool NTS, bool FULL>
__global__ __launch_bounds__((row_block_threads(TPR))) void sm_fwd_k(const float* __restrict__ x, float* __restrict__ y,
                                                                  int64_t rows, int H_arg) {
  const int H = FULL ? 4 * TPR * NV : H_arg;  // FULL: rows of exactly TPR * NV float4s
  constexpr int NT = row_block_threads(TPR);
  constexpr int GPB = NT / TPR;
  __shared__ float lds[2 * (NT / 64)];
  const int t = threadIdx.x % TPR;
  const int64_t row = (int64_t)blockIdx.x * GPB + threadIdx.x / TPR;
  if (row >= rows) return;
  const int h4 = H >> 2;
  RowTile<TPR, NV> xt;
  xt.load(x + row * H, h4, t);
  float m = NEG_INF;
#pragma unroll
  for (int k = 0; k < NV; ++k)
    if (k * TPR + t < h4) m = fmaxf(m, max4(xt.v[k]));
  m = group_max_once<TPR>(m, lds);  // one row per block: one barrier per reduction
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    if (k * TPR + t < h4) {
      const f4 z = xt.v[k] - m;
      const f4 e = exp4(z);
      s += sum4(e);
      xt.v[k] = LOG ? z : e;
    }
  }
  s = group_sum_once<TPR, float>(s, lds + NT / 64);
  if constexpr (LOG) {
    const float L = logf(s);
#pragma unroll
    for (int k = 0; k < NV; ++k) xt.v[k] = xt.v[k] - L;
  } else {
    div_by_sum<NV>(xt.v, s);  // e / s, rounded as the division operator rounds it
  }
  xt.template store<NTS>(y + row * H, h4, t);
}

template <int TPR, int NV, bool LOG, bool NTS, bool FULL>
__global__ __launch_bounds__((row_block_threads(TPR))) void sm_bwd_k(const float* __restrict__ y, const float* __restrict__ g,
                                                                  float* __restrict__ dx, int64_t rows, int H_arg) {
  const int H = FULL ? 4 * TPR * NV : H_arg;  // FULL: rows of exactly TPR * NV float4s
  constexpr int NT = row_block_threads(TPR);
  constexpr int GPB = NT / TPR;
  __shared__ float lds[NT / 64];
  const int t = threadIdx.x % TPR;
  const int64_t row = (int64_t)blockIdx.x * GPB + threadIdx.x / TPR;
  if (row >= rows) return;
  const int h4 = H >> 2;
  RowTile<TPR, NV> yt, gt;
  yt.load(y + row * H, h4, t);
  gt.load(g + row * H, h4, t);
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < NV; ++k) s += LOG ? sum4(gt.v[k]) : sum4(gt.v[k] * yt.v[k]);
  s = group_sum_once<TPR, float>(s, lds);  // the block's only reduction
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    if constexpr (LOG) gt.v[k] = gt.v[k] - exp4(yt.v[k]) * s;
    else gt.v[k] = yt.v[k] * (gt.v[k] - s);
  }
  gt.template store<NTS>(dx + row * H, h4, t);
}

// Last-dim kernels for any length / alignment: one block per row, two passes.
template <bool LOG>
__global__ __launch_bounds__(BS) void sm_fwd_loop_k(const float* __restrict__ x, float* __restrict__ y, int64_t rows, int H) {
  __shared__ float lds[2 * (BS / 64)];
  const int64_t row = blockIdx.x;
  const float* xr = x + row * H;
  Online o;
  for (int c = threadIdx.x; c < H; c += BS) o.add1(xr[c]);
  group_online<BS>(o, lds);
  float* yr = y + row * H;
  const float L = logf(o.s);
  for (int c = threadIdx.x; c < H; c += BS) {
    const float z = xr[c] - o.m;
    yr[c] = LOG ? z - L : expf(z) / o.s;
  }
}

template <bool LOG>
__global__ __launch_bounds__(BS) void sm_bwd_loop_k(const float* __restrict__ y, const float* __restrict__ g,
                                                    float* __restrict__ dx, int64_t rows, int H) {
  __shared__ float lds[BS / 64];
  const int64_t row = blockIdx.x;
  const float* yr = y + row * H;
  const float* gr = g + row * H;
  float s = 0.f;
  for (int c = threadIdx.x; c < H; c += BS) s += LOG ? gr[c] : gr[c] * yr[c];
  s = group_sum<BS, float>(s, lds);
  float* d = dx + row * H;
  for (int c = threadIdx.x; c < H; c += BS) d[c] = LOG ? gr[c] - expf(yr[c]) * s : yr[c] * (gr[c] - s);
}

// ---------------------------------------------------------------------------
// Middle-dim kernels (inner > 1): one thread per (o, i) column.

template <bool LOG>
__global__ __launch_bounds__(BS) void sm_fwd_col_k(const float* __restrict__ x, float* __restrict__ y,
                                                   int64_t outer, int64_t len, int64_t inner) {
  const int64_t id = (int64_t)blockIdx.x * BS + threadIdx.x;
  if (id >= outer * inner) return;
  const int64_t o = id / inner, i = id % inner;
  const float* xc = x + o * len * inner + i;
  float* yc = y + o * len * inner + i;
  Online st;
  for (int64_t k = 0; k < len; ++k) st.add1(xc[k * inner]);
  const float L = logf(st.s);
  for (int64_t k = 0; k < len; ++k) {
    const float z = xc[k * inner] - st.m;
    yc[k * inner] = LOG ? z - L : expf(z) / st.s;
  }
}

template <bool LOG>
__global__ __launch_bounds__(BS) void sm_bwd_col_k(const float* __restrict__ y, const float* __restrict__ g,
                                                   float* __restrict__ dx, int64_t outer, int64_t len, int64_t inner) {
  const int64_t id = (int64_t)blockIdx.x * BS + threadIdx.x;
  if (id >= outer * inner) return;
  const int64_t o = id / inner, i = id % inner;
  const int64_t base = o * len * inner + i;
  float s = 0.f;
  for (int64_t k = 0; k < len; ++k) {
    const int64_t p = base + k * inner;
    s += LOG ? g[p] : g[p] * y[p];
  }
  for (int64_t k = 0; k < len; ++k) {
    const int64_t p = base + k * inner;
    dx[p] = LOG ? g[p] - expf(y[p]) * s : y[p] * (g[p] - s);
  }
}

// ---------------------------------------------------------------------------
// Cross-entropy.

constexpr int CE_BS = 256;
constexpr int CE_U = 4;   // forward: float4 loads in flight per thread per step
constexpr int CE_BU = 1;  // backward: float4s per thread (one per thread streams fastest)

// The reference picks the target's log-probability as
// sum(onehot * log_softmax(x)) (functional.py:287-292): a non-target class
// whose log-probability is -inf (x - max == -inf: a -inf logit, or one so far
// below the max that the difference overflows) contributes 0 * -inf = NaN,
// so that row's picked value, and the loss, is NaN. `mn` is the row's
// minimum over its non-target logits; x - max is monotone in x.
__device__ __forceinline__ bool onehot_nan(float mn, float m) { return mn - m == NEG_INF; }

// v with component j replaced by +inf (out of a minimum).
__device__ __forceinline__ f4 drop_lane(const f4& v, int j) {
  const float P = -NEG_INF;
  return f4{j == 0 ? P : v.x, j == 1 ? P : v.y, j == 2 ? P : v.z, j == 3 ? P : v.w};
}

// Rows longer than the register-row kernel takes (more than 16384 float4s,
// or not vectorizable): one block per row, streaming it.
// lse[row] = max + log(sum exp(x - max));
// picked[row] = (x[t] - max) - log(sum)  (the reference's ls[row, t]), or
// NaN where the reference's one-hot product makes it NaN (onehot_nan).
__global__ __launch_bounds__(CE_BS) void ce_fwd_k(const float* __restrict__ logits, const int64_t* __restrict__ targets,
                                                  float* __restrict__ lse, float* __restrict__ picked, int64_t n, int C,
                                                  int vec, int* __restrict__ guard) {
  __shared__ float lds[2 * (CE_BS / 64)];
  const int64_t row = blockIdx.x;
  const float* xr = logits + row * C;
  int64_t tg = targets[row];
  const bool bad = tg < 0 || tg >= C;
  if (bad) tg = 0;
  float mn = -NEG_INF;
  Online o;
  if (vec) {
    const f4* p = reinterpret_cast<const f4*>(xr);
    const int c4 = C >> 2;
    const int ct = (int)(tg >> 2);
    const int jt = (int)(tg & 3);
    int c = threadIdx.x;
    for (; c + (CE_U - 1) * CE_BS < c4; c += CE_U * CE_BS) {
      f4 v[CE_U];
#pragma unroll
      for (int u = 0; u < CE_U; ++u) v[u] = ld_stream(p + c + u * CE_BS);
#pragma unroll
      for (int u = 0; u < CE_U; ++u) mn = fminf(mn, min4(c + u * CE_BS == ct ? drop_lane(v[u], jt) : v[u]));
      float cm = max4(v[0]);
#pragma unroll
      for (int u = 1; u < CE_U; ++u) cm = fmaxf(cm, max4(v[u]));
      if (cm > o.m) {
        o.s = (o.m == NEG_INF) ? 0.f : o.s * expf(o.m - cm);
        o.m = cm;
      }
      if (o.m != NEG_INF) {
        float acc = 0.f;
#pragma unroll
        for (int u = 0; u < CE_U; ++u) acc += sum4(exp4(v[u] - o.m));
        o.s += acc;
      } else {
#pragma unroll
        for (int u = 0; u < CE_U; ++u) o.add4(v[u]);
      }
    }
    for (; c < c4; c += CE_BS) {
      const f4 v = p[c];
      o.add4(v);
      mn = fminf(mn, min4(c == ct ? drop_lane(v, jt) : v));
    }
  } else {
    for (int c = threadIdx.x; c < C; c += CE_BS) {
      const float v = xr[c];
      o.add1(v);
      if (c != tg) mn = fminf(mn, v);
    }
  }
  group_online<CE_BS>(o, lds);
  mn = -group_max<CE_BS>(-mn, lds);
  if (threadIdx.x == 0) {
    if (bad) atomicOr(guard, 1);
    const float L = logf(o.s);
    lse[row] = o.m + L;
    picked[row] = onehot_nan(mn, o.m) ? __builtin_nanf("") : (xr[tg] - o.m) - L;
  }
}

// Rows of up to RT * NV float4s, a row per block held in registers, so each
// row crosses HBM once: the row max (with the non-target minimum that
// onehot_nan needs, in the same reduction) and the sum of e = exp(x - max)
// (two block reductions), lse and picked. With `dunit` set the block also writes, from
// the e it kept in the same registers, the gradient of the mean loss for an
// upstream gradient of exactly 1, as the composed log_softmax VJP forms it
// (functional.py:277-293 through ops.rs's exp/sum/log/sub VJPs):
// gS * e with gS = (1 / n) * (1 / s), and gS * e - 1 / n at the target, so a
// backward seeded with 1 has nothing left to compute. One exp per element:
// with a second exp(x - lse) for the gradient the kernel spent about 39 VALU
// instructions per element and ran at the VALU bound, not the HBM bound.
// The zero-sum residue the reference routes to the argmax (the max VJP) is
// rounding noise of the reference's own evaluation and is not formed.
// Measured at C3 (8192 x 32000), two-exp form: 512 x 16 ran the forward with
// the gradient in 380 us (1024 x 8, held to one block per CU by its 68 VGPRs:
// 476 us; 256 x 32: 417 us) and the forward alone in 181 us (streaming: 174 us).
// With one exp, the restructured loops below and 60 VGPRs, 1024 x 8 runs two
// blocks per CU and is the faster shape at C3 (see ce_forward).
// TAIL1: the row fills all but the last of a thread's NV float4 slots
// ((NV - 1) * RT < C / 4 <= NV * RT, as at C3's 32000 classes), so only slot
// NV - 1 is bounds-checked. The hot loops take the minimum over every logit;
// the reference's NaN rule needs the minimum over the non-target ones, which
// is formed again, with the target dropped, only for a row whose minimum
// could make it NaN. The target's logit comes from the owning thread's
// registers.
template <int RT, int NV, bool GRAD, bool NTS, bool TAIL1>
__global__ __launch_bounds__(RT) void ce_fwd_rows_k(const float* __restrict__ logits,
                                                    const int64_t* __restrict__ targets, float* __restrict__ lse,
                                                    float* __restrict__ picked, float* __restrict__ dunit, int64_t n,
                                                    int C, int* __restrict__ guard) {
  // slot sets: the max and the minimum, then the sum, then the rare
  // non-target minimum
  __shared__ float lds[4 * (RT / 64)];
  __shared__ float tlogit;
  const int64_t row = blockIdx.x;
  const int t = threadIdx.x;
  const int c4 = C >> 2;
  const float* xr = logits + row * C;
  const f4* p = reinterpret_cast<const f4*>(xr);
  auto in_row = [&](int k) { return (TAIL1 && k < NV - 1) || k * RT + t < c4; };
  f4 v[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int c = k * RT + t;
    v[k] = in_row(k) ? ld_stream(p + c) : f4{NEG_INF, NEG_INF, NEG_INF, NEG_INF};
  }
  int64_t tg = targets[row];
  const bool bad = tg < 0 || tg >= C;
  if (bad) tg = 0;
  // The target's float4 is slot kt of lane `own`; component jt.
  const int ct = (int)(tg >> 2);
  const int kt = ct / RT;
  const bool own = ct - kt * RT == t;
  const int jt = (int)(tg & 3);
  float m = NEG_INF;
  float mn = -NEG_INF;  // minimum over the row's logits (padding lanes hold -inf: skipped)
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    m = fmaxf(m, max4(v[k]));
    if (in_row(k)) mn = fminf(mn, min4(v[k]));
    if (k == kt) {
      if (own) tlogit = jt == 0 ? v[k].x : jt == 1 ? v[k].y : jt == 2 ? v[k].z : v[k].w;
    }
  }
  float nmn = -mn;
  group_max2_once<RT>(m, nmn, lds);
  const float ms = m == NEG_INF ? 0.f : m;
  // the row can be NaN only if its minimum is: then the minimum without the
  // target decides (block-uniform branch)
  bool nan_row = onehot_nan(-nmn, m);
  if (nan_row) {
    float mt = -NEG_INF;
#pragma unroll
    for (int k = 0; k < NV; ++k)
      if (in_row(k)) mt = fminf(mt, min4(k == kt && own ? drop_lane(v[k], jt) : v[k]));
    float nmt = -mt;
    nmt = group_max_once<RT>(nmt, lds + 3 * (RT / 64));
    nan_row = onehot_nan(-nmt, m);
  }
  // Lanes past the row hold -inf: their e is exp(-inf) = 0 and adds nothing.
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    v[k] = exp4(v[k] - ms);
    s += sum4(v[k]);
  }
  s = group_sum_once<RT, float>(s, lds + 2 * (RT / 64));  // its barrier also publishes tlogit
  if constexpr (RT == 64) __syncthreads();                 // (one wave: no barrier in the reduction)
  const float L = logf(s);
  if (t == 0) {
    if (bad) atomicOr(guard, 1);
    lse[row] = m + L;
    picked[row] = nan_row ? __builtin_nanf("") : (tlogit - m) - L;
  }
  if constexpr (GRAD) {
    const float scale = 1.0f / (float)n;
    const float gs = scale * (1.0f / s);
    f4* q = reinterpret_cast<f4*>(dunit + row * C);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int c = k * RT + t;
      if (in_row(k)) {
        f4 d = v[k] * gs;
        if (k == kt) {
          if (own) {
            if (jt == 0) d.x -= scale;
            else if (jt == 1) d.y -= scale;
            else if (jt == 2) d.z -= scale;
            else d.w -= scale;
          }
        }
        st_stream<NTS>(d, q + c);
      }
    }
  }
}

// loss[0] = -(sum(picked) / n), sum in float64 in fixed order.
__global__ __launch_bounds__(1024) void ce_mean_k(const float* __restrict__ picked, int64_t n, float* __restrict__ loss) {
  __shared__ double s[1024];
  double acc = 0.0;
  for (int64_t i = threadIdx.x; i < n; i += 1024) acc += (double)picked[i];
  s[threadIdx.x] = acc;
  __syncthreads();
  for (int w = 512; w >= 1; w >>= 1) {
    if ((int)threadIdx.x < w) s[threadIdx.x] += s[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) loss[0] = -((float)s[0] / (float)n);
}

// dlogits = (exp(x - lse) - onehot) * (g / n). Grid: (column blocks, rows).
template <bool NTS>
__global__ __launch_bounds__(CE_BS) void ce_bwd_k(const float* __restrict__ logits, const int64_t* __restrict__ targets,
                                                  const float* __restrict__ lse, const float* __restrict__ gloss,
                                                  float* __restrict__ dlogits, int64_t n, int C, int vec) {
  const int64_t row = blockIdx.y;
  const float scale = gloss[0] / (float)n;
  const float l = lse[row];
  int64_t t = targets[row];
  const float* xr = logits + row * C;
  float* dr = dlogits + row * C;
  if (vec) {
    const f4* p = reinterpret_cast<const f4*>(xr);
    f4* q = reinterpret_cast<f4*>(dr);
    const int c4 = C >> 2;
    const int per_block = CE_BS * CE_BU;
    const int c0 = blockIdx.x * per_block + threadIdx.x;
    f4 v[CE_BU];
#pragma unroll
    for (int u = 0; u < CE_BU; ++u) {
      const int c = c0 + u * CE_BS;
      if (c < c4) v[u] = ld_stream(p + c);
    }
#pragma unroll
    for (int u = 0; u < CE_BU; ++u) {
      const int c = c0 + u * CE_BS;
      if (c < c4) {
        f4 e = exp4(v[u] - l);
        const int64_t base = (int64_t)c * 4;
        if (t >= base && t < base + 4) {
          const int j = (int)(t - base);
          if (j == 0) e.x -= 1.f;
          else if (j == 1) e.y -= 1.f;
          else if (j == 2) e.z -= 1.f;
          else e.w -= 1.f;
        }
        st_stream<NTS>(e * scale, q + c);
      }
    }
  } else {
    const int per_block = CE_BS * CE_BU;
    const int c0 = blockIdx.x * per_block + threadIdx.x;
    for (int u = 0; u < CE_BU; ++u) {
      const int c = c0 + u * CE_BS;
      if (c < C) {
        float e = expf(xr[c] - l);
        if (c == t) e -= 1.f;
        dr[c] = e * scale;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Host dispatch.


bool aligned16(std::initializer_list<const void*> ps) {
  for (const void* p : ps)
    if (reinterpret_cast<uintptr_t>(p) & 15u) return false;
  return true;
}

int check_olen(const char* what, int64_t outer, int64_t len, int64_t inner, std::initializer_list<const void*> ps) {
  if (outer < 0 || len < 0 || inner < 0)
    return fail(OXI_INVALID_ARGUMENT, "%s: negative size", what);
  // len and outer * inner each bounded, and the element count inside int64
  const int64_t lim = (int64_t)1 << 40;
  if (len > ((int64_t)1 << 30) || (outer && inner > lim / outer) ||
      (outer && inner && len > (((int64_t)1 << 60) / outer) / inner))
    return fail(OXI_INVALID_ARGUMENT, "%s: size exceeds the kernel limits", what);
  if (outer && len && inner)
    for (const void* p : ps)
      if (!p) return fail(OXI_INVALID_ARGUMENT, "%s: NULL tensor pointer", what);
  return OXI_OK;
}

template <bool LOG>
int launch_fwd(const float* x, float* y, int64_t outer, int64_t len, int64_t inner) {
  hipStream_t s = stream();
  if (inner == 1) {
    const int cfg = (len % 4 == 0 && aligned16({x, y})) ? pick_row_cfg(len / 4) : 0;
    const int h = (int)len;
    const bool nts = nt_stores(outer * len * 4);
#define OXI_SMF_GO(TPR, NV, NTS, FULL)                                                                  \
  sm_fwd_k<TPR, NV, LOG, NTS, FULL><<<dim3((unsigned)ceil_div(outer, row_block_threads(TPR) / TPR)),         \
                                     dim3(row_block_threads(TPR)), 0, s>>>(x, y, outer, h)
#define OXI_SMF(TPR, NV)                                                                                   \
  case TPR * 10 + NV:                                                                                      \
    if (h == 4 * TPR * NV) {                                                                               \
      if (nts) OXI_SMF_GO(TPR, NV, true, true);                                                            \
      else OXI_SMF_GO(TPR, NV, false, true);                                                               \
    } else {                                                                                               \
      if (nts) OXI_SMF_GO(TPR, NV, true, false);                                                           \
      else OXI_SMF_GO(TPR, NV, false, false);                                                              \
    }                                                                                                      \
    break;
    switch (cfg) {
      OXI_SMF(64, 1)
      OXI_SMF(64, 2)
      OXI_SMF(64, 3)
      OXI_SMF(64, 4)
      OXI_SMF(256, 2)
      OXI_SMF(256, 4)
      OXI_SMF(256, 8)
                default:
        sm_fwd_loop_k<LOG><<<dim3((unsigned)outer), dim3(BS), 0, s>>>(x, y, outer, h);
    }
#undef OXI_SMF
#undef OXI_SMF_GO
  } else {
    sm_fwd_col_k<LOG><<<dim3((unsigned)ceil_div(outer * inner, BS)), dim3(BS), 0, s>>>(x, y, outer, len, inner);
  }
  return check_launch(LOG ? "log_softmax_fwd" : "softmax_fwd");
}

template <bool LOG>
int launch_bwd(const float* y, const float* g, float* dx, int64_t outer, int64_t len, int64_t inner) {
  hipStream_t s = stream();
  if (inner == 1) {
    const int cfg = (len % 4 == 0 && aligned16({y, g, dx})) ? pick_row_cfg(len / 4) : 0;
    const int h = (int)len;
    const bool nts = nt_stores(outer * len * 4);
#define OXI_SMB_GO(TPR, NV, NTS, FULL)                                                                  \
  sm_bwd_k<TPR, NV, LOG, NTS, FULL><<<dim3((unsigned)ceil_div(outer, row_block_threads(TPR) / TPR)),         \
                                     dim3(row_block_threads(TPR)), 0, s>>>(y, g, dx, outer, h)
#define OXI_SMB(TPR, NV)                                                                                   \
  case TPR * 10 + NV:                                                                                      \
    if (h == 4 * TPR * NV) {                                                                               \
      if (nts) OXI_SMB_GO(TPR, NV, true, true);                                                            \
      else OXI_SMB_GO(TPR, NV, false, true);                                                               \
    } else {                                                                                               \
      if (nts) OXI_SMB_GO(TPR, NV, true, false);                                                           \
      else OXI_SMB_GO(TPR, NV, false, false);                                                              \
    }                                                                                                      \
    break;
    switch (cfg) {
      OXI_SMB(64, 1)
      OXI_SMB(64, 2)
      OXI_SMB(64, 3)
      OXI_SMB(64, 4)
      OXI_SMB(256, 2)
      OXI_SMB(256, 4)
      OXI_SMB(256, 8)
                default:
        sm_bwd_loop_k<LOG><<<dim3((unsigned)outer), dim3(BS), 0, s>>>(y, g, dx, outer, h);
    }
#undef OXI_SMB
#undef OXI_SMB_GO
  } else {
    sm_bwd_col_k<LOG><<<dim3((unsigned)ceil_div(outer * inner, BS)), dim3(BS), 0, s>>>(y, g, dx, outer, len, inner);
  }
  return check_launch(LOG ? "log_softmax_bwd" : "softmax_bwd");
}

}  // namespace
}  // namespace oxi

using namespace oxi;

extern "C" {

int oxi_softmax_fwd(const float* x, float* y, int64_t outer, int64_t len, int64_t inner) {
  if (int rc = check_olen("softmax_fwd", outer, len, inner, {x, y})) return rc;
  if (outer == 0 || inner == 0 || len == 0) return OXI_OK;
  OXI_CHECK_INIT();
  return launch_fwd<false>(x, y, outer, len, inner);
}

int oxi_softmax_bwd(const float* y, const float* g, float* dx, int64_t outer, int64_t len, int64_t inner) {
  if (int rc = check_olen("softmax_bwd", outer, len, inner, {y, g, dx})) return rc;
  if (outer == 0 || inner == 0 || len == 0) return OXI_OK;
  OXI_CHECK_INIT();
  return launch_bwd<false>(y, g, dx, outer, len, inner);
}

int oxi_log_softmax_fwd(const float* x, float* y, int64_t outer, int64_t len, int64_t inner) {
  if (int rc = check_olen("log_softmax_fwd", outer, len, inner, {x, y})) return rc;
  if (outer == 0 || inner == 0 || len == 0) return OXI_OK;
  OXI_CHECK_INIT();
  return launch_fwd<true>(x, y, outer, len, inner);
}

int oxi_log_softmax_bwd(const float* y, const float* g, float* dx, int64_t outer, int64_t len, int64_t inner) {
  if (int rc = check_olen("log_softmax_bwd", outer, len, inner, {y, g, dx})) return rc;
  if (outer == 0 || inner == 0 || len == 0) return OXI_OK;
  OXI_CHECK_INIT();
  return launch_bwd<true>(y, g, dx, outer, len, inner);
}

}  // extern "C"

namespace oxi {
namespace {

// Loss and lse; with `dunit`, also the gradient for an upstream 1 (rows of
// c % 4 == 0 with 16-byte aligned operands only: NOT_IMPLEMENTED otherwise,
// before anything is launched).
int ce_forward(const char* what, const float* logits, const int64_t* targets, float* loss, float* lse, float* dunit,
               int64_t n, int64_t c) {
  if (n < 0 || c < 0) return fail(OXI_INVALID_ARGUMENT, "%s: negative size", what);
  if (!loss) return fail(OXI_INVALID_ARGUMENT, "%s: loss must not be NULL", what);
  if (c > ((int64_t)1 << 30) || n > ((int64_t)1 << 31) - 1)
    return fail(OXI_INVALID_ARGUMENT, "%s: size exceeds the kernel limits", what);
  OXI_CHECK_INIT();
  // picked.mean() of no rows: reduce_all's Mean of an empty strip is 0
  // (bindings lib.rs:126-143, ops.rs:247-249), and the loss is its negation
  if (n == 0) return oxi_fill(loss, 1, -0.0f);
  if (c == 0) return fail(OXI_INVALID_ARGUMENT, "%s: zero classes", what);
  if (!logits || !targets || !lse) return fail(OXI_INVALID_ARGUMENT, "%s: NULL tensor pointer", what);
  const int vec = (c % 4 == 0 && aligned16({logits})) ? 1 : 0;
  const int64_t c4 = c / 4;
  // (threads, float4s a thread) of the register-row kernel: 16 float4s a
  // thread, as few threads as the row needs; rows of 4097 to 8192 float4s
  // take 1024 threads of 8 (60 VGPRs, two blocks per CU): C3's step 362.6
  // and 362.7 us against 367.3 and 367.9 at 512 x 16 on one box.
  int rt = 0, nv = 16;
  if (vec) {
    if (c4 > 4096 && c4 <= 8192) {
      rt = 1024;
      nv = 8;
    } else {
      for (int t = 64; t <= 1024 && !rt; t *= 2)
        if (c4 <= (int64_t)t * 16) rt = t;
    }
  }
  if (dunit && !(rt && aligned16({dunit})))
    return fail(OXI_NOT_IMPLEMENTED, "%s: rows of %lld classes do not take the one-pass kernel (c %% 4 != 0, more "
                "than 65536 classes or unaligned)", what, (long long)c);
  Workspace picked(sizeof(float) * (size_t)n);
  if (!picked.p) return fail_alloc("cross_entropy_fwd: workspace");
  const dim3 grid((unsigned)n);
  float* pk = picked.as<float>();
  const bool nt = nt_stores(n * c * 4);  // the gradient's stores
  switch (rt * 100 + nv) {
#define OXI_CE_GO(RT, NV, GRAD, NTS, TAIL1)                                                                \
  ce_fwd_rows_k<RT, NV, GRAD, NTS, TAIL1><<<grid, dim3(RT), 0, stream()>>>(logits, targets, lse, pk, dunit, n, \
                                                                          (int)c, guard_flag())
#define OXI_CE_ROWS(RT, NV)                                                                                 \
  case RT * 100 + NV:                                                                                       \
    if (c4 > (NV - 1) * RT) {                                                                               \
      if (!dunit) OXI_CE_GO(RT, NV, false, false, true);                                                    \
      else if (nt) OXI_CE_GO(RT, NV, true, true, true);                                                     \
      else OXI_CE_GO(RT, NV, true, false, true);                                                            \
    } else {                                                                                                \
      if (!dunit) OXI_CE_GO(RT, NV, false, false, false);                                                   \
      else if (nt) OXI_CE_GO(RT, NV, true, true, false);                                                    \
      else OXI_CE_GO(RT, NV, true, false, false);                                                           \
    }                                                                                                       \
    break;
    OXI_CE_ROWS(64, 16)
    OXI_CE_ROWS(128, 16)
    OXI_CE_ROWS(256, 16)
    OXI_CE_ROWS(1024, 8)
    OXI_CE_ROWS(1024, 16)
#undef OXI_CE_ROWS
#undef OXI_CE_GO
    default:
      ce_fwd_k<<<grid, dim3(CE_BS), 0, stream()>>>(logits, targets, lse, pk, n, (int)c, vec, guard_flag());
  }
  if (int rc = check_launch(what)) return rc;
  ce_mean_k<<<1, 1024, 0, stream()>>>(picked.as<float>(), n, loss);
  return check_launch("cross_entropy_mean");
}

}  // namespace
}  // namespace oxi

extern "C" {

int oxi_cross_entropy_fwd(const float* logits, const int64_t* targets, float* loss, float* lse, int64_t n, int64_t c) {
  return ce_forward("cross_entropy_fwd", logits, targets, loss, lse, nullptr, n, c);
}

int oxi_cross_entropy_fwd_grad(const float* logits, const int64_t* targets, float* loss, float* lse, float* dlogits,
                               int64_t n, int64_t c) {
  if (!dlogits && n > 0 && c > 0) return fail(OXI_INVALID_ARGUMENT, "cross_entropy_fwd_grad: NULL dlogits");
  return ce_forward("cross_entropy_fwd_grad", logits, targets, loss, lse, n > 0 && c > 0 ? dlogits : nullptr, n, c);
}

int oxi_cross_entropy_bwd(const float* logits, const int64_t* targets, const float* lse, const float* gloss,
                          float* dlogits, int64_t n, int64_t c) {
  if (n < 0 || c < 0) return fail(OXI_INVALID_ARGUMENT, "cross_entropy_bwd: negative size");
  if (c > ((int64_t)1 << 30) || n > 65535LL * 32768LL)
    return fail(OXI_INVALID_ARGUMENT, "cross_entropy_bwd: size exceeds the kernel limits");
  if (n == 0 || c == 0) return OXI_OK;
  if (!logits || !targets || !lse || !gloss || !dlogits)
    return fail(OXI_INVALID_ARGUMENT, "cross_entropy_bwd: NULL tensor pointer");
  OXI_CHECK_INIT();
  const int vec = (c % 4 == 0 && aligned16({logits, dlogits})) ? 1 : 0;
  const int64_t units = vec ? c / 4 : c;
  const unsigned gx = (unsigned)ceil_div(units, CE_BS * CE_BU);
  const bool nts = nt_stores(n * c * 4);
  if (n > 65535) {
    // grid.y is limited; launch row slabs
    for (int64_t r0 = 0; r0 < n; r0 += 65535) {
      const int64_t nr = (n - r0) < 65535 ? (n - r0) : 65535;
      if (nts)
        ce_bwd_k<true><<<dim3(gx, (unsigned)nr), dim3(CE_BS), 0, stream()>>>(logits + r0 * c, targets + r0, lse + r0,
                                                                             gloss, dlogits + r0 * c, n, (int)c, vec);
      else
        ce_bwd_k<false><<<dim3(gx, (unsigned)nr), dim3(CE_BS), 0, stream()>>>(logits + r0 * c, targets + r0, lse + r0,
                                                                              gloss, dlogits + r0 * c, n, (int)c, vec);
      if (int rc = check_launch("cross_entropy_bwd")) return rc;
    }
    return OXI_OK;
  }
  if (nts) ce_bwd_k<true><<<dim3(gx, (unsigned)n), dim3(CE_BS), 0, stream()>>>(logits, targets, lse, gloss, dlogits, n, (int)c, vec);
  else ce_bwd_k<false><<<dim3(gx, (unsigned)n), dim3(CE_BS), 0, stream()>>>(logits, targets, lse, gloss, dlogits, n, (int)c, vec);
  return check_launch("cross_entropy_bwd");
}

}  // extern "C"
