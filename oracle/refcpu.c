/*
 * refcpu.c -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.
 *
 * A plain-C restatement of the oxitorch reference CPU path for the
 * layer-kernel hot path, used only as the parity checker by tests/, by
 * __graft_entry__.smoke() and as the timed CPU baseline of bench.py. Nothing in
 * oxitorch_amd/ links, loads or calls it.
 *
 * The reference (Rust, crates/ + python/oxitorch) cannot be built here (no
 * cargo/rustc, crates not vendored), so this file re-executes the same op
 * graph in f32 with the same rounding order:
 *   - every elementwise op rounds on its own (build with -ffp-contract=off);
 *   - row/strip sums are sequential f32 folds (ReduceKind::reduce_strip,
 *     crates/oxi-tensor/src/ops.rs:246-285), mean = sum / len in f32;
 *   - broadcast gradients are reduced as graph::unbroadcast does
 *     (crates/oxi-autograd/src/graph.rs:274-313): one prepended axis at a
 *     time, each a sequential column fold;
 *   - gradient contributions are accumulated in the reverse topological order
 *     of graph::topo_order / backward_ext (graph.rs:324-438), derived per
 *     composition in the comments below;
 *   - libm expf/logf/tanhf/powf, as Rust's f32::{exp,ln,tanh,powf} lower to.
 * Each function cites the reference lines it restates.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define EXPORT __attribute__((visibility("default")))

/* ---- helpers ------------------------------------------------------------ */

/* sequential f32 fold of a strip: ReduceKind::Sum (ops.rs:256) */
static float seq_sum(const float* p, int64_t n, int64_t stride) {
  float s = 0.0f;
  for (int64_t i = 0; i < n; ++i) s += p[i * stride];
  return s;
}

/* graph::unbroadcast (graph.rs:274-313) of a contiguous (lead..., H) tensor `v`
 * down to (H,): sums prepended axis 0 repeatedly (keepdim), each a serial
 * column fold (Tensor::reduce non-last-dim path, crates/oxi-tensor/src/lib.rs:549-558). */
static void unbroadcast_lead(const float* v, const int64_t* lead, int nlead, int64_t H, float* out) {
  int64_t rest = 1;
  for (int i = 0; i < nlead; ++i) rest *= lead[i];
  if (nlead == 0) {
    memcpy(out, v, sizeof(float) * (size_t)H);
    return;
  }
  float* cur = (float*)malloc(sizeof(float) * (size_t)(rest * H));
  memcpy(cur, v, sizeof(float) * (size_t)(rest * H));
  for (int a = 0; a < nlead; ++a) {
    const int64_t len = lead[a];
    const int64_t inner = rest / len * H;  /* elements after axis a (current layout) */
    for (int64_t i = 0; i < inner; ++i) {
      float s = 0.0f;
      for (int64_t k = 0; k < len; ++k) s += cur[k * inner + i];
      cur[i] = s;
    }
    rest /= len;
  }
  memcpy(out, cur, sizeof(float) * (size_t)H);
  free(cur);
}

/* ---- F.rms_norm (python/oxitorch/nn/functional.py:236-240) -------------- */

/* ms = (x*x).mean(-1, True); inv = (ms + eps).apply("rsqrt"); y = (x*inv)*w */
EXPORT void ref_rms_norm_fwd(const float* x, const float* w, float* y, float* inv, int64_t rows, int64_t H,
                             float eps) {
  float* sq = (float*)malloc(sizeof(float) * (size_t)H);
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * H;
    for (int64_t c = 0; c < H; ++c) sq[c] = xr[c] * xr[c];
    const float ms = seq_sum(sq, H, 1) / (float)H;          /* Mean strip, ops.rs:257 */
    const float iv = 1.0f / sqrtf(ms + eps);                 /* rsqrt, ops.rs:138-141 */
    inv[r] = iv;
    for (int64_t c = 0; c < H; ++c) y[r * H + c] = (xr[c] * iv) * w[c];
  }
  free(sq);
}

/* Reference VJP: inv is detached (bindings lib.rs:682-710), so the graph is
 * y = mul(mul(x, inv), w):  dx = (g*w)*inv ; dw = unbroadcast(g * (x*inv)). */
EXPORT void ref_rms_norm_bwd(const float* x, const float* w, const float* inv, const float* g, float* dx,
                             float* dw, const int64_t* lead, int nlead, int64_t H) {
  int64_t rows = 1;
  for (int i = 0; i < nlead; ++i) rows *= lead[i];
  float* gb = (float*)malloc(sizeof(float) * (size_t)(rows * H));
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < H; ++c) {
      const int64_t i = r * H + c;
      const float a = x[i] * inv[r];
      gb[i] = g[i] * a;                       /* mul VJP gb = g*a (ops.rs:65-72) */
      if (dx) dx[i] = (g[i] * w[c]) * inv[r]; /* ga = g*w, then ga*inv */
    }
  if (dw) unbroadcast_lead(gb, lead, nlead, H, dw);
  free(gb);
}

/* ---- F.layer_norm (functional.py:227-233) -------------------------------- */

EXPORT void ref_layer_norm_fwd(const float* x, const float* w, const float* b, float* y, float* mean, float* inv,
                               int64_t rows, int64_t H, float eps) {
  float* c = (float*)malloc(sizeof(float) * (size_t)H);
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * H;
    const float mu = seq_sum(xr, H, 1) / (float)H;
    for (int64_t k = 0; k < H; ++k) c[k] = xr[k] - mu;
    float s = 0.0f;
    for (int64_t k = 0; k < H; ++k) s += c[k] * c[k];
    const float var = s / (float)H;
    const float iv = 1.0f / sqrtf(var + eps);
    mean[r] = mu;
    inv[r] = iv;
    for (int64_t k = 0; k < H; ++k) y[r * H + k] = ((c[k] * iv) * w[k]) + b[k];
  }
  free(c);
}

/* Reference VJP (inv detached). Graph: c = sub(x, mu); mu = mean(x);
 * out = add(mul(mul(c, inv), w), b). Reverse topological order: add, mul(.,w),
 * mul(c,inv), sub, mean. So x.grad = gc (from sub) + (sum(-gc) * (1/H)) (from
 * mean: ops.rs:341-348 multiplies by the f32 1/n), gc = (g*w)*inv;
 * dw = unbroadcast(g*(c*inv)), db = unbroadcast(g). */
EXPORT void ref_layer_norm_bwd(const float* x, const float* w, const float* mean, const float* inv, const float* g,
                               float* dx, float* dw, float* db, const int64_t* lead, int nlead, int64_t H) {
  int64_t rows = 1;
  for (int i = 0; i < nlead; ++i) rows *= lead[i];
  float* gb = (float*)malloc(sizeof(float) * (size_t)(rows * H));
  float* gc = (float*)malloc(sizeof(float) * (size_t)H);
  const float inv_n = 1.0f / (float)H;
  for (int64_t r = 0; r < rows; ++r) {
    float neg_sum = 0.0f;
    for (int64_t k = 0; k < H; ++k) {
      const int64_t i = r * H + k;
      const float c = x[i] - mean[r];
      gb[i] = g[i] * (c * inv[r]);
      gc[k] = (g[i] * w[k]) * inv[r];
      neg_sum += -gc[k];                      /* sub VJP: unbroadcast(-g) over the row */
    }
    const float corr = neg_sum * inv_n;       /* mean VJP: expand, mul_scalar(1/n) */
    if (dx)
      for (int64_t k = 0; k < H; ++k) dx[r * H + k] = gc[k] + corr;
  }
  if (dw) unbroadcast_lead(gb, lead, nlead, H, dw);
  if (db) unbroadcast_lead(g, lead, nlead, H, db);
  free(gb);
  free(gc);
}

/* ---- F.gelu tanh approximation (functional.py:194-199) ------------------ */

static const float GELU_K = 0.044715f;
static const float GELU_C = (float)0.7978845608028654; /* float(np.sqrt(2/np.pi)) as f32 */

EXPORT void ref_gelu_tanh_fwd(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    const float v = x[i];
    const float x32 = v * v;
    const float t1 = v * x32;
    const float t2 = t1 * GELU_K;
    const float t3 = v + t2;
    const float inner = t3 * GELU_C;
    const float th = tanhf(inner);
    const float op = th + 1.0f;  /* 1.0 + t -> add(t, full(1)) */
    const float hx = v * 0.5f;   /* 0.5 * x -> mul(x, full(0.5)) */
    y[i] = hx * op;
  }
}

/* Composed VJP. Nodes: x32=x*x, t1=x*x32, t2=t1*K, t3=x+t2, inner=t3*C,
 * th=tanh(inner), op=th+1, hx=x*0.5, y=hx*op. topo_order (graph.rs:324-349)
 * from y gives, reversed: y, hx, op, th, inner, t3, t2, t1, x32, so x.grad
 * accumulates: hx branch, t3 branch, t1 branch, then both x32 operands. */
EXPORT void ref_gelu_tanh_bwd(const float* x, const float* g, float* dx, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    const float v = x[i];
    const float x32 = v * v;
    const float t1 = v * x32;
    const float t2 = t1 * GELU_K;
    const float t3 = v + t2;
    const float inner = t3 * GELU_C;
    const float th = tanhf(inner);
    const float op = th + 1.0f;
    const float hx = v * 0.5f;
    const float g_hx = g[i] * op;
    const float g_op = g[i] * hx;
    const float th2 = tanhf(inner) * tanhf(inner); /* tanh VJP recomputes (ops.rs:218-230) */
    const float g_inner = g_op * (1.0f - th2);
    const float g_t3 = g_inner * GELU_C;
    const float g_t1 = g_t3 * GELU_K;
    const float g_x32 = g_t1 * v;
    float acc = g_hx * 0.5f;
    acc = acc + g_t3;
    acc = acc + g_t1 * x32;
    acc = acc + g_x32 * v;
    acc = acc + g_x32 * v;
    dx[i] = acc;
  }
}

/* ---- F.silu (functional.py:202-204): x * sigmoid(x) --------------------- */

static float sigmoidf_ref(float a) { return 1.0f / (1.0f + expf(-a)); } /* ops.rs:174-177 */

EXPORT void ref_silu_fwd(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = x[i] * sigmoidf_ref(x[i]);
}

/* Reverse topo: mul (x.grad = g*s), then sigmoid (x.grad += (g*x)*(s*(1-s))). */
EXPORT void ref_silu_bwd(const float* x, const float* g, float* dx, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    const float s = sigmoidf_ref(x[i]);
    const float a = g[i] * s;
    const float gs = g[i] * x[i];
    dx[i] = a + gs * (s * (1.0f - s));
  }
}

/* ---- softmax / log_softmax over the middle dim of (outer, len, inner) ---- */

/* max fold: fold(-inf, f32::max) (ops.rs:258); argmax: strict > from index 0 (ops.rs:261-270) */
static void strip_max_arg(const float* p, int64_t len, int64_t st, float* m, int64_t* arg) {
  float mv = -INFINITY;
  for (int64_t k = 0; k < len; ++k) mv = fmaxf(mv, p[k * st]);
  int64_t best = 0;
  float bv = p[0];
  for (int64_t k = 0; k < len; ++k)
    if (p[k * st] > bv) {
      bv = p[k * st];
      best = k;
    }
  *m = mv;
  *arg = best;
}

/* softmax (functional.py:211-215): m = x.max(dim,True); e = exp(x-m); y = e / e.sum(dim,True) */
EXPORT void ref_softmax_fwd(const float* x, float* y, int64_t outer, int64_t len, int64_t inner) {
  for (int64_t o = 0; o < outer; ++o)
    for (int64_t i = 0; i < inner; ++i) {
      const float* xs = x + o * len * inner + i;
      float* ys = y + o * len * inner + i;
      float m;
      int64_t arg;
      strip_max_arg(xs, len, inner, &m, &arg);
      float s = 0.0f;
      for (int64_t k = 0; k < len; ++k) s += expf(xs[k * inner] - m);
      for (int64_t k = 0; k < len; ++k) ys[k * inner] = expf(xs[k * inner] - m) / s;
    }
}

/* Composed VJP. Reverse topo: div(e, s), sum(e), exp(z), sub(x, m), max(x).
 * div: ge = g/s ; gs = unbroadcast(-((g*e)/(s*s))) (ops.rs:80-91)
 * sum: e.grad += expand(gs) ; exp: gz = e.grad * exp(z)
 * sub: x.grad = gz, m.grad = sum(-gz) ; max: x.grad[argmax] += m.grad (ops.rs:350-370). */
EXPORT void ref_softmax_bwd(const float* x, const float* g, float* dx, int64_t outer, int64_t len, int64_t inner) {
  float* e = (float*)malloc(sizeof(float) * (size_t)len);
  float* gz = (float*)malloc(sizeof(float) * (size_t)len);
  for (int64_t o = 0; o < outer; ++o)
    for (int64_t i = 0; i < inner; ++i) {
      const float* xs = x + o * len * inner + i;
      const float* gsrc = g + o * len * inner + i;
      float* d = dx + o * len * inner + i;
      float m;
      int64_t arg;
      strip_max_arg(xs, len, inner, &m, &arg);
      float s = 0.0f;
      for (int64_t k = 0; k < len; ++k) {
        e[k] = expf(xs[k * inner] - m);
        s += e[k];
      }
      const float s2 = s * s;
      float gsum = 0.0f;
      for (int64_t k = 0; k < len; ++k) gsum += -((gsrc[k * inner] * e[k]) / s2);
      float msum = 0.0f;
      for (int64_t k = 0; k < len; ++k) {
        const float eg = (gsrc[k * inner] / s) + gsum;
        gz[k] = eg * expf(xs[k * inner] - m);
        msum += -gz[k];
      }
      for (int64_t k = 0; k < len; ++k) d[k * inner] = gz[k] + (k == arg ? msum : 0.0f);
    }
  free(e);
  free(gz);
}

/* log_softmax (functional.py:218-222): z = x - max; y = z - log(sum(exp z)) */
EXPORT void ref_log_softmax_fwd(const float* x, float* y, int64_t outer, int64_t len, int64_t inner) {
  for (int64_t o = 0; o < outer; ++o)
    for (int64_t i = 0; i < inner; ++i) {
      const float* xs = x + o * len * inner + i;
      float* ys = y + o * len * inner + i;
      float m;
      int64_t arg;
      strip_max_arg(xs, len, inner, &m, &arg);
      float s = 0.0f;
      for (int64_t k = 0; k < len; ++k) s += expf(xs[k * inner] - m);
      const float L = logf(s);
      for (int64_t k = 0; k < len; ++k) ys[k * inner] = (xs[k * inner] - m) - L;
    }
}

/* Composed VJP. Reverse topo: sub(z, L) [z.grad = g, L.grad = sum(-g)],
 * log(S) [S.grad = L.grad * (1/S)], sum(e) [e.grad = expand], exp(z)
 * [z.grad += e.grad*exp(z)], sub(x, m) [x.grad = z.grad, m.grad = sum(-z.grad)],
 * max [x.grad[argmax] += m.grad]. */
EXPORT void ref_log_softmax_bwd(const float* x, const float* g, float* dx, int64_t outer, int64_t len,
                                int64_t inner) {
  float* zg = (float*)malloc(sizeof(float) * (size_t)len);
  for (int64_t o = 0; o < outer; ++o)
    for (int64_t i = 0; i < inner; ++i) {
      const float* xs = x + o * len * inner + i;
      const float* gsrc = g + o * len * inner + i;
      float* d = dx + o * len * inner + i;
      float m;
      int64_t arg;
      strip_max_arg(xs, len, inner, &m, &arg);
      float s = 0.0f;
      for (int64_t k = 0; k < len; ++k) s += expf(xs[k * inner] - m);
      float lg = 0.0f;
      for (int64_t k = 0; k < len; ++k) lg += -gsrc[k * inner];
      const float gS = lg * (1.0f / s);
      float msum = 0.0f;
      for (int64_t k = 0; k < len; ++k) {
        const float z = xs[k * inner] - m;
        zg[k] = gsrc[k * inner] + gS * expf(z);
        msum += -zg[k];
      }
      for (int64_t k = 0; k < len; ++k) d[k * inner] = zg[k] + (k == arg ? msum : 0.0f);
    }
  free(zg);
}

/* ---- F.cross_entropy, mean (functional.py:277-293) ----------------------- */

/* ls = log_softmax(logits); picked = (onehot*ls).sum(-1); loss = -(picked.mean()).
 * targets already resolved to [0, c). Writes the scalar loss. */
EXPORT void ref_cross_entropy_fwd(const float* logits, const int64_t* targets, float* loss, int64_t n, int64_t c) {
  float* ls = (float*)malloc(sizeof(float) * (size_t)c);
  float psum = 0.0f;
  for (int64_t r = 0; r < n; ++r) {
    ref_log_softmax_fwd(logits + r * c, ls, 1, c, 1);
    float picked = 0.0f;
    for (int64_t k = 0; k < c; ++k) picked += (k == targets[r] ? 1.0f : 0.0f) * ls[k];
    psum += picked;
  }
  /* picked.mean(): reduce_all (bindings lib.rs:126-143) reduces with
   * reduce_strip, whose Mean of an empty strip is 0 (ops.rs:247-249), so an
   * empty batch gives -(0.0) = -0.0 */
  const float mean = n > 0 ? psum / (float)n : 0.0f;
  *loss = -mean;
  free(ls);
}

/* Composed VJP with upstream gloss: neg -> -gloss; mean -> * (1/n) (f32);
 * sum(-1) -> expand; mul(onehot, ls) -> g_ls = g * onehot; then the
 * log_softmax VJP above. */
EXPORT void ref_cross_entropy_bwd(const float* logits, const int64_t* targets, float gloss, float* dlogits, int64_t n,
                                  int64_t c) {
  float* gl = (float*)malloc(sizeof(float) * (size_t)c);
  const float gmean = (-gloss) * (1.0f / (float)n);
  for (int64_t r = 0; r < n; ++r) {
    for (int64_t k = 0; k < c; ++k) gl[k] = gmean * (k == targets[r] ? 1.0f : 0.0f);
    ref_log_softmax_bwd(logits + r * c, gl, dlogits + r * c, 1, c, 1);
  }
  free(gl);
}

/* ---- index_select / embedding (crates/oxi-tensor/src/lib.rs:665-703) ----- */

/* Returns 0, or 1 when an index is out of range (nothing written then). */
EXPORT int ref_index_select(const float* src, int64_t outer, int64_t len, int64_t inner, const int64_t* idx, int64_t n,
                            float* out) {
  for (int64_t k = 0; k < n; ++k) {
    const int64_t i = idx[k] < 0 ? len + idx[k] : idx[k];
    if (i < 0 || i >= len) return 1;
  }
  for (int64_t o = 0; o < outer; ++o)
    for (int64_t k = 0; k < n; ++k) {
      const int64_t i = idx[k] < 0 ? len + idx[k] : idx[k];
      memcpy(out + (o * n + k) * inner, src + (o * len + i) * inner, sizeof(float) * (size_t)inner);
    }
  return 0;
}

/* scatter_index_select (crates/oxi-autograd/src/ops.rs:741-769): zeros, then
 * data[(o*len+idx)*inner+i] += g[(o*n+k)*inner+i] in position order k. */
EXPORT void ref_index_select_bwd(const float* g, int64_t outer, int64_t len, int64_t inner, const int64_t* idx,
                                 int64_t n, float* grad) {
  memset(grad, 0, sizeof(float) * (size_t)(outer * len * inner));
  for (int64_t o = 0; o < outer; ++o)
    for (int64_t k = 0; k < n; ++k) {
      const int64_t v = idx[k] < 0 ? len + idx[k] : idx[k];
      float* d = grad + (o * len + v) * inner;
      const float* s = g + (o * n + k) * inner;
      for (int64_t i = 0; i < inner; ++i) d[i] += s[i];
    }
}

/* ---- dim reductions (Tensor::reduce, lib.rs:519-576; reduce_strip, ops.rs:246-285) */

/* kind: 0 sum, 1 mean, 2 max, 3 min, 4 argmax, 5 argmin, 6 norm. x contiguous.
 * Returns 0, or 1 for max/min/arg* over an empty dim. */
EXPORT int ref_reduce(int kind, const float* x, const int64_t* shape, int ndim, int dim, float* out) {
  int64_t outer = 1, inner = 1;
  for (int d = 0; d < dim; ++d) outer *= shape[d];
  for (int d = dim + 1; d < ndim; ++d) inner *= shape[d];
  const int64_t len = shape[dim];
  if (len == 0 && kind >= 2 && kind <= 5) return 1;
  for (int64_t o = 0; o < outer; ++o)
    for (int64_t i = 0; i < inner; ++i) {
      const float* p = x + o * len * inner + i;
      float r = 0.0f;
      if (len == 0) {
        out[o * inner + i] = 0.0f;
        continue;
      }
      switch (kind) {
        case 0: r = seq_sum(p, len, inner); break;
        case 1: r = seq_sum(p, len, inner) / (float)len; break;
        case 2: { float m = -INFINITY; for (int64_t k = 0; k < len; ++k) m = fmaxf(m, p[k * inner]); r = m; } break;
        case 3: { float m = INFINITY; for (int64_t k = 0; k < len; ++k) m = fminf(m, p[k * inner]); r = m; } break;
        case 4: { int64_t b = 0; float bv = p[0]; for (int64_t k = 0; k < len; ++k) if (p[k * inner] > bv) { bv = p[k * inner]; b = k; } r = (float)b; } break;
        case 5: { int64_t b = 0; float bv = p[0]; for (int64_t k = 0; k < len; ++k) if (p[k * inner] < bv) { bv = p[k * inner]; b = k; } r = (float)b; } break;
        default: { float s = 0.0f; for (int64_t k = 0; k < len; ++k) s += p[k * inner] * p[k * inner]; r = sqrtf(s); } break;
      }
      out[o * inner + i] = r;
    }
  return 0;
}

/* ---- elementwise registry (crates/oxi-tensor/src/ops.rs:55-202) ---------- */

EXPORT void ref_unary(int op, const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    const float a = x[i];
    float r;
    switch (op) {
      case 0: r = -a; break;
      case 1: r = fabsf(a); break;
      case 2: r = sqrtf(a); break;
      case 3: r = 1.0f / sqrtf(a); break;
      case 4: r = expf(a); break;
      case 5: r = logf(a); break;
      case 6: r = log2f(a); break;
      case 7: r = log10f(a); break;
      case 8: r = sinf(a); break;
      case 9: r = cosf(a); break;
      case 10: r = tanhf(a); break;
      case 11: r = fmaxf(a, 0.0f); break;
      case 12: r = sigmoidf_ref(a); break;
      case 13: r = floorf(a); break;
      case 14: r = ceilf(a); break;
      case 15: r = roundf(a); break;
      case 16: r = isnan(a) ? a : copysignf(1.0f, a); break;
      case 17: r = a * a; break;
      case 18: r = 1.0f / a; break;
      default: r = a; break;
    }
    y[i] = r;
  }
}

/* Row-major walk of `shape` with broadcast strides for a and b (iterate::map_n). */
EXPORT void ref_binary(int op, const float* a, const int64_t* as, const float* b, const int64_t* bs, float* y,
                       const int64_t* shape, int ndim) {
  int64_t n = 1;
  for (int d = 0; d < ndim; ++d) n *= shape[d];
  int64_t idx[16] = {0};
  for (int64_t e = 0; e < n; ++e) {
    int64_t oa = 0, ob = 0;
    for (int d = 0; d < ndim; ++d) {
      oa += idx[d] * as[d];
      ob += idx[d] * bs[d];
    }
    const float u = a[oa], v = b[ob];
    float r;
    switch (op) {
      case 0: r = u + v; break;
      case 1: r = u - v; break;
      case 2: r = u * v; break;
      case 3: r = u / v; break;
      case 4: r = powf(u, v); break;
      case 5: r = fminf(u, v); break;
      case 6: r = fmaxf(u, v); break;
      case 7: r = u == v; break;
      case 8: r = u != v; break;
      case 9: r = u < v; break;
      case 10: r = u <= v; break;
      case 11: r = u > v; break;
      default: r = u >= v; break;
    }
    y[e] = r;
    for (int d = ndim - 1; d >= 0; --d) {
      if (++idx[d] < shape[d]) break;
      idx[d] = 0;
    }
  }
}

/* ---- exact-erf GELU: NOT in the reference (its F.gelu is the tanh form,
 * functional.py:194-199). Closed form evaluated in f32 with libm erff/expf,
 * used as the CPU baseline of config 2; parity is pinned by the float64
 * closed form (oracle/closed_form.py). ------------------------------------ */

EXPORT void ref_gelu_erf_fwd(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = (0.5f * x[i]) * (1.0f + erff(x[i] * 0.70710678118654752f));
}

EXPORT void ref_gelu_erf_bwd(const float* x, const float* g, float* dx, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    const float v = x[i];
    const float cdf = 0.5f * (1.0f + erff(v * 0.70710678118654752f));
    const float pdf = expf(-0.5f * (v * v)) * 0.3989422804014327f;
    dx[i] = g[i] * (cdf + v * pdf);
  }
}

/* ---- optimizer steps (crates/oxi-autograd/src/optim.rs) ------------------ */

/* Sgd::step_param (optim.rs:104-137) for one parameter with a gradient:
 * buf = momentum*buf + g (buf starts at zeros, optim.rs:113-115);
 * update = nesterov ? g + momentum*buf : buf, or g without momentum;
 * p_out = p - lr*update. `buf` may be NULL when momentum == 0. */
EXPORT void ref_sgd_step(const float* p, const float* g, float* buf, float* p_out, int64_t n, float lr, float momentum,
                         int nesterov) {
  for (int64_t i = 0; i < n; ++i) {
    float upd = g[i];
    if (momentum > 0.0f) {
      buf[i] = momentum * buf[i] + g[i];
      upd = nesterov ? g[i] + momentum * buf[i] : buf[i];
    }
    p_out[i] = p[i] - lr * upd;
  }
}

/* AdamW::step_param (optim.rs:223-262) for one parameter with a gradient at
 * step t: bc1 = 1 - beta1^t, bc2 = 1 - beta2^t in f32 powf (optim.rs:233-234);
 * classic Adam (decoupled = 0) folds weight_decay*p into the gradient, AdamW
 * subtracts lr*weight_decay*p after the adaptive step. */
EXPORT void ref_adamw_step(const float* p, const float* g, float* m, float* v, float* p_out, int64_t n, float lr,
                           float beta1, float beta2, float eps, float weight_decay, int decoupled, int64_t t) {
  const float bc1 = 1.0f - powf(beta1, (float)t);
  const float bc2 = 1.0f - powf(beta2, (float)t);
  for (int64_t i = 0; i < n; ++i) {
    const float val = p[i];
    const float ge = (!decoupled && weight_decay != 0.0f) ? g[i] + weight_decay * val : g[i];
    m[i] = beta1 * m[i] + (1.0f - beta1) * ge;
    v[i] = beta2 * v[i] + (1.0f - beta2) * ge * ge;
    const float mh = m[i] / bc1;
    const float vh = v[i] / bc2;
    float next = val - lr * mh / (sqrtf(vh) + eps);
    if (decoupled && weight_decay != 0.0f) next -= lr * weight_decay * val;
    p_out[i] = next;
  }
}

/* ---- scatter_dim0 (Tensor::scatter_dim0, crates/oxi-tensor/src/lib.rs:895-932) */

/* out = base (rows, inner) with row idx[p] replaced by values[p] for p in
 * order (last write wins). Returns 0, or 1 when an index is out of range
 * (checked before anything is written, lib.rs:912-919). */
EXPORT int ref_scatter_dim0(const float* base, int64_t rows, int64_t inner, const int64_t* idx, int64_t n,
                            const float* values, float* out) {
  for (int64_t p = 0; p < n; ++p) {
    const int64_t r = idx[p] < 0 ? rows + idx[p] : idx[p];
    if (r < 0 || r >= rows) return 1;
  }
  memcpy(out, base, sizeof(float) * (size_t)(rows * inner));
  for (int64_t p = 0; p < n; ++p) {
    const int64_t r = idx[p] < 0 ? rows + idx[p] : idx[p];
    memcpy(out + r * inner, values + p * inner, sizeof(float) * (size_t)inner);
  }
  return 0;
}

/* VJP of aops::scatter_dim0 (crates/oxi-autograd/src/ops.rs:531-600):
 * gbase = g * mask with mask 0 on every written row and 1 elsewhere
 * (a multiply, so a negative g gives -0 on written rows); slot p of gvalues
 * gets g's row idx[p] when p is that row's last writer, zeros otherwise.
 * Either output may be NULL. */
EXPORT void ref_scatter_dim0_bwd(const float* g, int64_t rows, int64_t inner, const int64_t* idx, int64_t n,
                                 float* gbase, float* gvalues) {
  int64_t* last = (int64_t*)malloc(sizeof(int64_t) * (size_t)(rows > 0 ? rows : 1));
  for (int64_t r = 0; r < rows; ++r) last[r] = -1;
  for (int64_t p = 0; p < n; ++p) last[idx[p] < 0 ? rows + idx[p] : idx[p]] = p;
  if (gbase)
    for (int64_t r = 0; r < rows; ++r) {
      const float m = last[r] >= 0 ? 0.0f : 1.0f;
      for (int64_t i = 0; i < inner; ++i) gbase[r * inner + i] = g[r * inner + i] * m;
    }
  if (gvalues)
    for (int64_t p = 0; p < n; ++p) {
      const int64_t r = idx[p] < 0 ? rows + idx[p] : idx[p];
      for (int64_t i = 0; i < inner; ++i) gvalues[p * inner + i] = last[r] == p ? g[r * inner + i] : 0.0f;
    }
  free(last);
}

/* ---- masked_select (Tensor::masked_select, lib.rs:939-961) ------------------ */

/* Row-major walk of the broadcast `shape` (iterate::map_n): an element is
 * picked when its mask value != 0; the reference marks unpicked elements NaN
 * and then drops every NaN, so a picked NaN of x is dropped too. Writes the
 * picks to `out` (capacity: the grid size) and returns their count. */
EXPORT int64_t ref_masked_select(const float* x, const int64_t* xs, const float* m, const int64_t* ms,
                                 const int64_t* shape, int ndim, float* out) {
  int64_t n = 1;
  for (int d = 0; d < ndim; ++d) n *= shape[d];
  int64_t idx[16] = {0};
  int64_t cnt = 0;
  for (int64_t e = 0; e < n; ++e) {
    int64_t ox = 0, om = 0;
    for (int d = 0; d < ndim; ++d) {
      ox += idx[d] * xs[d];
      om += idx[d] * ms[d];
    }
    const float v = m[om] == 0.0f ? NAN : x[ox];
    if (!isnan(v)) out[cnt++] = v;
    for (int d = ndim - 1; d >= 0; --d) {
      if (++idx[d] < shape[d]) break;
      idx[d] = 0;
    }
  }
  return cnt;
}

/* VJP of aops::masked_select (crates/oxi-autograd/src/ops.rs:609-667): walk
 * the same grid; each point whose mask value != 0 takes the next upstream
 * gradient and adds it to x's element at gx_strides (row-major strides of x's
 * own shape, 0 on broadcast dims), starting from zeros. The picks are counted
 * from the mask alone (ops.rs:650-653). Mask strides: row-major of the mask's
 * own shape, 0 on broadcast dims (ops.rs:628-640). */
EXPORT void ref_masked_select_bwd(const float* m, const int64_t* ms, const int64_t* shape, int ndim, const float* g,
                                  float* gx, const int64_t* gx_strides, int64_t x_numel) {
  for (int64_t i = 0; i < x_numel; ++i) gx[i] = 0.0f;
  int64_t n = 1;
  for (int d = 0; d < ndim; ++d) n *= shape[d];
  int64_t idx[16] = {0};
  int64_t pick = 0;
  for (int64_t e = 0; e < n; ++e) {
    int64_t om = 0, ox = 0;
    for (int d = 0; d < ndim; ++d) {
      om += idx[d] * ms[d];
      ox += idx[d] * gx_strides[d];
    }
    if (m[om] != 0.0f) gx[ox] += g[pick++];
    for (int d = ndim - 1; d >= 0; --d) {
      if (++idx[d] < shape[d]) break;
      idx[d] = 0;
    }
  }
}
