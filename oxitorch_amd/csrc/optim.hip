// Optimizer steps on flat device slices: SGD with optional (Nesterov)
// momentum and Adam/AdamW (crates/oxi-autograd/src/optim.rs:104-137,
// 223-262). One float4 per thread (the fastest streaming shape on MI355X);
// every product and sum rounds on its own in the reference's order (the
// library builds with -ffp-contract=off), division and sqrt are IEEE, so a
// step matches the reference's f32 loop bit for bit.
//
// The new parameter values go to `p_out`, which may be `p` itself (each
// element is read, then written, by the same thread). Optimizer state
// (`buf`, `m`, `v`) is updated in place.
#include <cmath>

#include "internal.h"
#include "rowtile.h"

namespace oxi {
namespace {

constexpr int BS = 256;

struct SgdArgs {
  float lr, momentum;
  int nesterov;
};

__device__ __forceinline__ float sgd_elem(float p, float g, float* b, const SgdArgs& a) {
  float upd = g;
  if (a.momentum > 0.0f) {
    const float nb = a.momentum * *b + g;
    *b = nb;
    upd = a.nesterov ? g + a.momentum * nb : nb;
  }
  return p - a.lr * upd;
}

template <bool VEC, bool NTS>
__global__ __launch_bounds__(BS) void sgd_k(const float* p, const float* __restrict__ g, float* __restrict__ buf,
                                            float* p_out, int64_t n, SgdArgs a) {
  const int64_t i = (int64_t)blockIdx.x * BS + threadIdx.x;
  if constexpr (VEC) {
    if (i >= (n >> 2)) return;
    const f4 pv = ld_stream(reinterpret_cast<const f4*>(p) + i);
    const f4 gv = ld_stream(reinterpret_cast<const f4*>(g) + i);
    f4 bv = a.momentum > 0.0f ? ld_stream(reinterpret_cast<const f4*>(buf) + i) : f4{0.f, 0.f, 0.f, 0.f};
    f4 r;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float b = bv[c];
      r[c] = sgd_elem(pv[c], gv[c], &b, a);
      bv[c] = b;
    }
    if (a.momentum > 0.0f) st_stream<NTS>(bv, reinterpret_cast<f4*>(buf) + i);
    st_stream<NTS>(r, reinterpret_cast<f4*>(p_out) + i);
  } else {
    if (i >= n) return;
    float b = a.momentum > 0.0f ? buf[i] : 0.0f;
    const float r = sgd_elem(p[i], g[i], &b, a);
    if (a.momentum > 0.0f) buf[i] = b;
    p_out[i] = r;
  }
}

struct AdamArgs {
  float lr, beta1, beta2, eps, wd, bc1, bc2;
  int decoupled;
};

__device__ __forceinline__ float adam_elem(float val, float g, float* m, float* v, const AdamArgs& a) {
  const float ge = (!a.decoupled && a.wd != 0.0f) ? g + a.wd * val : g;
  const float nm = a.beta1 * *m + (1.0f - a.beta1) * ge;
  const float nv = a.beta2 * *v + (1.0f - a.beta2) * ge * ge;
  *m = nm;
  *v = nv;
  const float mh = nm / a.bc1;
  const float vh = nv / a.bc2;
  float next = val - a.lr * mh / (sqrtf(vh) + a.eps);
  if (a.decoupled && a.wd != 0.0f) next -= a.lr * a.wd * val;
  return next;
}

template <bool VEC, bool NTS>
__global__ __launch_bounds__(BS) void adam_k(const float* p, const float* __restrict__ g, float* __restrict__ m,
                                             float* __restrict__ v, float* p_out, int64_t n, AdamArgs a) {
  const int64_t i = (int64_t)blockIdx.x * BS + threadIdx.x;
  if constexpr (VEC) {
    if (i >= (n >> 2)) return;
    const f4 pv = ld_stream(reinterpret_cast<const f4*>(p) + i);
    const f4 gv = ld_stream(reinterpret_cast<const f4*>(g) + i);
    f4 mv = ld_stream(reinterpret_cast<const f4*>(m) + i);
    f4 vv = ld_stream(reinterpret_cast<const f4*>(v) + i);
    f4 r;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float mc = mv[c], vc = vv[c];
      r[c] = adam_elem(pv[c], gv[c], &mc, &vc, a);
      mv[c] = mc;
      vv[c] = vc;
    }
    st_stream<NTS>(mv, reinterpret_cast<f4*>(m) + i);
    st_stream<NTS>(vv, reinterpret_cast<f4*>(v) + i);
    st_stream<NTS>(r, reinterpret_cast<f4*>(p_out) + i);
  } else {
    if (i >= n) return;
    float mc = m[i], vc = v[i];
    p_out[i] = adam_elem(p[i], g[i], &mc, &vc, a);
    m[i] = mc;
    v[i] = vc;
  }
}

// ---- multi-tensor steps ------------------------------------------------------
// One launch covers up to MT_MAX parameters; their descriptors travel in the
// kernel arguments (no device table, no copy). Block b serves the slice s with
// block_end[s-1] <= b < block_end[s] (a uniform binary search over the
// argument array), one float4 unit per thread; a slice's last unit handles
// its n % 4 tail elementwise. Every pointer must be 16-byte aligned.
constexpr int MT_MAX = 32;

template <int NPTR>
struct MultiArgs {
  float* ptr[NPTR][MT_MAX];  // operand k of slice s
  int64_t n[MT_MAX];
  float bc1[MT_MAX], bc2[MT_MAX];
  uint32_t block_end[MT_MAX];
  int count;
};

template <int NPTR>
__device__ __forceinline__ int find_slice(const MultiArgs<NPTR>& a, uint32_t b) {
  int lo = 0, hi = a.count - 1;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (b < a.block_end[mid]) hi = mid;
    else lo = mid + 1;
  }
  return lo;
}

// p, g, buf, out
template <bool NTS>
__global__ __launch_bounds__(BS) void sgd_multi_k(MultiArgs<4> a, SgdArgs h) {
  const int s = find_slice(a, blockIdx.x);
  const uint32_t first = s ? a.block_end[s - 1] : 0u;
  const int64_t u = (int64_t)(blockIdx.x - first) * BS + threadIdx.x;
  const int64_t n = a.n[s];
  const int64_t e0 = u * 4;
  if (e0 >= n) return;
  const float* p = a.ptr[0][s];
  const float* g = a.ptr[1][s];
  float* buf = a.ptr[2][s];
  float* out = a.ptr[3][s];
  if (e0 + 4 <= n) {
    const f4 pv = ld_stream(reinterpret_cast<const f4*>(p) + u);
    const f4 gv = ld_stream(reinterpret_cast<const f4*>(g) + u);
    f4 bv = h.momentum > 0.0f ? ld_stream(reinterpret_cast<const f4*>(buf) + u) : f4{0.f, 0.f, 0.f, 0.f};
    f4 r;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float b = bv[c];
      r[c] = sgd_elem(pv[c], gv[c], &b, h);
      bv[c] = b;
    }
    if (h.momentum > 0.0f) st_stream<NTS>(bv, reinterpret_cast<f4*>(buf) + u);
    st_stream<NTS>(r, reinterpret_cast<f4*>(out) + u);
  } else {
    for (int64_t e = e0; e < n; ++e) {
      float b = h.momentum > 0.0f ? buf[e] : 0.0f;
      const float r = sgd_elem(p[e], g[e], &b, h);
      if (h.momentum > 0.0f) buf[e] = b;
      out[e] = r;
    }
  }
}

// p, g, m, v, out
template <bool NTS>
__global__ __launch_bounds__(BS) void adam_multi_k(MultiArgs<5> a, AdamArgs h) {
  const int s = find_slice(a, blockIdx.x);
  const uint32_t first = s ? a.block_end[s - 1] : 0u;
  const int64_t u = (int64_t)(blockIdx.x - first) * BS + threadIdx.x;
  const int64_t n = a.n[s];
  const int64_t e0 = u * 4;
  if (e0 >= n) return;
  h.bc1 = a.bc1[s];
  h.bc2 = a.bc2[s];
  const float* p = a.ptr[0][s];
  const float* g = a.ptr[1][s];
  float* m = a.ptr[2][s];
  float* v = a.ptr[3][s];
  float* out = a.ptr[4][s];
  if (e0 + 4 <= n) {
    const f4 pv = ld_stream(reinterpret_cast<const f4*>(p) + u);
    const f4 gv = ld_stream(reinterpret_cast<const f4*>(g) + u);
    f4 mv = ld_stream(reinterpret_cast<const f4*>(m) + u);
    f4 vv = ld_stream(reinterpret_cast<const f4*>(v) + u);
    f4 r;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float mc = mv[c], vc = vv[c];
      r[c] = adam_elem(pv[c], gv[c], &mc, &vc, h);
      mv[c] = mc;
      vv[c] = vc;
    }
    st_stream<NTS>(mv, reinterpret_cast<f4*>(m) + u);
    st_stream<NTS>(vv, reinterpret_cast<f4*>(v) + u);
    st_stream<NTS>(r, reinterpret_cast<f4*>(out) + u);
  } else {
    for (int64_t e = e0; e < n; ++e) {
      float mc = m[e], vc = v[e];
      out[e] = adam_elem(p[e], g[e], &mc, &vc, h);
      m[e] = mc;
      v[e] = vc;
    }
  }
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// grid x (blocks * threads) stays below 2^32 work-items
bool fits_grid(int64_t units) { return ceil_div(units, BS) * BS <= (int64_t)0xFFFFFFFFu; }

// float4 path for the largest multiple of 4, scalar kernel for the rest
// (launched on the same stream, disjoint elements).
template <class K4, class K1>
int launch_split(int64_t n, bool vec, K4 k4, K1 k1, const char* what) {
  const int64_t n4 = vec ? (n >> 2) : 0;
  if (n4 > 0) k4((unsigned)ceil_div(n4, BS), n4 * 4);
  const int64_t done = n4 * 4;
  if (done < n) k1((unsigned)ceil_div(n - done, BS), done, n - done);
  return check_launch(what);
}

}  // namespace
}  // namespace oxi

using namespace oxi;

extern "C" {

int oxi_sgd_step(const float* p, const float* g, float* buf, float* p_out, int64_t n, float lr, float momentum,
                 int nesterov) {
  if (n < 0) return fail(OXI_INVALID_ARGUMENT, "sgd_step: negative size");
  if (nesterov && !(momentum > 0.0f)) return fail(OXI_INVALID_ARGUMENT, "nesterov momentum requires momentum > 0");
  if (n == 0) return OXI_OK;
  if (!p || !g || !p_out) return fail(OXI_INVALID_ARGUMENT, "sgd_step: NULL tensor pointer");
  if (momentum > 0.0f && !buf) return fail(OXI_INVALID_ARGUMENT, "sgd_step: momentum needs a state buffer");
  if (!fits_grid(ceil_div(n, 4))) return fail(OXI_INVALID_ARGUMENT, "sgd_step: size exceeds the kernel limits");
  OXI_CHECK_INIT();
  hipStream_t s = stream();
  const SgdArgs a{lr, momentum, nesterov ? 1 : 0};
  const bool vec = al16(p) && al16(g) && al16(p_out) && (momentum <= 0.0f || al16(buf));
  const bool nts = nt_stores(n * 4 * (momentum > 0.0f ? 2 : 1));
  return launch_split(
      n, vec,
      [&](unsigned blocks, int64_t nn) {
        if (nts) sgd_k<true, true><<<blocks, BS, 0, s>>>(p, g, buf, p_out, nn, a);
        else sgd_k<true, false><<<blocks, BS, 0, s>>>(p, g, buf, p_out, nn, a);
      },
      [&](unsigned blocks, int64_t off, int64_t nn) {
        sgd_k<false, false><<<blocks, BS, 0, s>>>(p + off, g + off, buf ? buf + off : nullptr, p_out + off, nn, a);
      },
      "sgd_step");
}

int oxi_adamw_step(const float* p, const float* g, float* m, float* v, float* p_out, int64_t n, float lr, float beta1,
                   float beta2, float eps, float weight_decay, int decoupled, int64_t t) {
  if (n < 0) return fail(OXI_INVALID_ARGUMENT, "adamw_step: negative size");
  if (t < 1) return fail(OXI_INVALID_ARGUMENT, "adamw_step: step count must be >= 1 (got %lld)", (long long)t);
  if (n == 0) return OXI_OK;
  if (!p || !g || !m || !v || !p_out) return fail(OXI_INVALID_ARGUMENT, "adamw_step: NULL tensor pointer");
  if (!fits_grid(ceil_div(n, 4))) return fail(OXI_INVALID_ARGUMENT, "adamw_step: size exceeds the kernel limits");
  OXI_CHECK_INIT();
  hipStream_t s = stream();
  // bias corrections in f32 powf, as the reference (optim.rs:233-234)
  AdamArgs a{lr, beta1, beta2, eps, weight_decay, 1.0f - powf(beta1, (float)t), 1.0f - powf(beta2, (float)t),
             decoupled ? 1 : 0};
  const bool vec = al16(p) && al16(g) && al16(m) && al16(v) && al16(p_out);
  const bool nts = nt_stores(n * 4 * 3);
  return launch_split(
      n, vec,
      [&](unsigned blocks, int64_t nn) {
        if (nts) adam_k<true, true><<<blocks, BS, 0, s>>>(p, g, m, v, p_out, nn, a);
        else adam_k<true, false><<<blocks, BS, 0, s>>>(p, g, m, v, p_out, nn, a);
      },
      [&](unsigned blocks, int64_t off, int64_t nn) {
        adam_k<false, false><<<blocks, BS, 0, s>>>(p + off, g + off, m + off, v + off, p_out + off, nn, a);
      },
      "adamw_step");
}

int oxi_sgd_step_multi(const oxi_sgd_slice* slices, int count, float lr, float momentum, int nesterov) {
  if (count < 0) return fail(OXI_INVALID_ARGUMENT, "sgd_step_multi: negative slice count");
  if (nesterov && !(momentum > 0.0f)) return fail(OXI_INVALID_ARGUMENT, "nesterov momentum requires momentum > 0");
  if (count > 0 && !slices) return fail(OXI_INVALID_ARGUMENT, "sgd_step_multi: NULL slice array");
  const bool mom = momentum > 0.0f;
  int64_t bytes = 0;
  for (int i = 0; i < count; ++i) {
    const oxi_sgd_slice& q = slices[i];
    if (q.n < 0) return fail(OXI_INVALID_ARGUMENT, "sgd_step_multi: slice %d has a negative size", i);
    if (q.n == 0) continue;
    if (!q.p || !q.g || !q.p_out || (mom && !q.buf))
      return fail(OXI_INVALID_ARGUMENT, "sgd_step_multi: slice %d has a NULL pointer", i);
    if (!fits_grid(ceil_div(q.n, 4))) return fail(OXI_INVALID_ARGUMENT, "sgd_step_multi: slice %d is too large", i);
    bytes += q.n * 4 * (mom ? 2 : 1);
  }
  if (bytes == 0) return OXI_OK;
  OXI_CHECK_INIT();
  hipStream_t s = stream();
  const SgdArgs h{lr, momentum, nesterov ? 1 : 0};
  const bool nts = nt_stores(bytes);
  MultiArgs<4> a{};
  int64_t blocks = 0;
  auto flush = [&]() {
    if (!a.count) return;
    if (nts) sgd_multi_k<true><<<(unsigned)blocks, BS, 0, s>>>(a, h);
    else sgd_multi_k<false><<<(unsigned)blocks, BS, 0, s>>>(a, h);
    a.count = 0;
    blocks = 0;
  };
  for (int i = 0; i < count; ++i) {
    const oxi_sgd_slice& q = slices[i];
    if (q.n == 0) continue;
    if (!al16(q.p) || !al16(q.g) || !al16(q.p_out) || (mom && !al16(q.buf))) {
      const int rc = oxi_sgd_step(q.p, q.g, q.buf, q.p_out, q.n, lr, momentum, nesterov);
      if (rc != OXI_OK) return rc;
      continue;
    }
    const int64_t nb = ceil_div(ceil_div(q.n, 4), BS);
    if (a.count == MT_MAX || (blocks + nb) * BS > (int64_t)0xFFFFFFFFu) flush();
    const int k = a.count++;
    a.ptr[0][k] = const_cast<float*>(q.p);
    a.ptr[1][k] = const_cast<float*>(q.g);
    a.ptr[2][k] = q.buf;
    a.ptr[3][k] = q.p_out;
    a.n[k] = q.n;
    blocks += nb;
    a.block_end[k] = (uint32_t)blocks;
  }
  flush();
  return check_launch("sgd_step_multi");
}

int oxi_adamw_step_multi(const oxi_adamw_slice* slices, int count, float lr, float beta1, float beta2, float eps,
                         float weight_decay, int decoupled) {
  if (count < 0) return fail(OXI_INVALID_ARGUMENT, "adamw_step_multi: negative slice count");
  if (count > 0 && !slices) return fail(OXI_INVALID_ARGUMENT, "adamw_step_multi: NULL slice array");
  int64_t bytes = 0;
  for (int i = 0; i < count; ++i) {
    const oxi_adamw_slice& q = slices[i];
    if (q.n < 0) return fail(OXI_INVALID_ARGUMENT, "adamw_step_multi: slice %d has a negative size", i);
    if (q.t < 1) return fail(OXI_INVALID_ARGUMENT, "adamw_step_multi: slice %d: step count must be >= 1", i);
    if (q.n == 0) continue;
    if (!q.p || !q.g || !q.m || !q.v || !q.p_out)
      return fail(OXI_INVALID_ARGUMENT, "adamw_step_multi: slice %d has a NULL pointer", i);
    if (!fits_grid(ceil_div(q.n, 4))) return fail(OXI_INVALID_ARGUMENT, "adamw_step_multi: slice %d is too large", i);
    bytes += q.n * 4 * 3;
  }
  if (bytes == 0) return OXI_OK;
  OXI_CHECK_INIT();
  hipStream_t s = stream();
  const AdamArgs h{lr, beta1, beta2, eps, weight_decay, 1.0f, 1.0f, decoupled ? 1 : 0};
  const bool nts = nt_stores(bytes);
  MultiArgs<5> a{};
  int64_t blocks = 0;
  auto flush = [&]() {
    if (!a.count) return;
    if (nts) adam_multi_k<true><<<(unsigned)blocks, BS, 0, s>>>(a, h);
    else adam_multi_k<false><<<(unsigned)blocks, BS, 0, s>>>(a, h);
    a.count = 0;
    blocks = 0;
  };
  for (int i = 0; i < count; ++i) {
    const oxi_adamw_slice& q = slices[i];
    if (q.n == 0) continue;
    if (!al16(q.p) || !al16(q.g) || !al16(q.m) || !al16(q.v) || !al16(q.p_out)) {
      const int rc = oxi_adamw_step(q.p, q.g, q.m, q.v, q.p_out, q.n, lr, beta1, beta2, eps, weight_decay, decoupled,
                                    q.t);
      if (rc != OXI_OK) return rc;
      continue;
    }
    const int64_t nb = ceil_div(ceil_div(q.n, 4), BS);
    if (a.count == MT_MAX || (blocks + nb) * BS > (int64_t)0xFFFFFFFFu) flush();
    const int k = a.count++;
    a.ptr[0][k] = const_cast<float*>(q.p);
    a.ptr[1][k] = const_cast<float*>(q.g);
    a.ptr[2][k] = q.m;
    a.ptr[3][k] = q.v;
    a.ptr[4][k] = q.p_out;
    a.n[k] = q.n;
    // bias corrections in f32 powf per parameter step count (optim.rs:233-234)
    a.bc1[k] = 1.0f - powf(beta1, (float)q.t);
    a.bc2[k] = 1.0f - powf(beta2, (float)q.t);
    blocks += nb;
    a.block_end[k] = (uint32_t)blocks;
  }
  flush();
  return check_launch("adamw_step_multi");
}

}  // extern "C"
