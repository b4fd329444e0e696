// Differentiable ops: restates crates/oxi-autograd/src/ops.rs over device
// tensors, plus the fused hot-path nodes (one graph node and one kernel per
// direction for rms_norm, layer_norm, gelu, silu, softmax/log_softmax,
// cross_entropy and the embedding gather).
//
// Gradients produced inside VJPs keep the common dense layout of their
// operands (result_strides): a gradient flowing through a permuted view stays
// permuted, so the permute VJP hands the next node a contiguous tensor.
#include <atomic>
#include <cstdlib>
#include <cstring>

#include "host.h"

namespace oxt {
namespace aops {

namespace {

using Grads = std::vector<std::optional<Tensor>>;

Tensor un(int op, const Tensor& a) { return t_unary(op, a, true); }
Tensor bin(int op, const Tensor& a, const Tensor& b) { return t_binary(op, a, b, true); }
Tensor ones_of(const Tensor& t) { return t_scalar_full(t.shape, 1.0f, t.dev()); }

}  // namespace

// ---- binary (ops.rs:37-114) -------------------------------------------------------

Var add(const Var& a, const Var& b) {
  Tensor out = t_binary(OXI_BINARY_ADD, a.value(), b.value());
  return Var::op(out, "add", {a, b}, [](const Tensor& g, const std::vector<bool>& need) -> Grads {
    return {need[0] ? std::optional<Tensor>(g) : std::nullopt, need[1] ? std::optional<Tensor>(g) : std::nullopt};
  });
}

Var sub(const Var& a, const Var& b) {
  Tensor out = t_binary(OXI_BINARY_SUB, a.value(), b.value());
  return Var::op(out, "sub", {a, b}, [](const Tensor& g, const std::vector<bool>& need) -> Grads {
    Grads r(2);
    if (need[0]) r[0] = g;
    if (need[1]) r[1] = un(OXI_UNARY_NEG, g);
    return r;
  });
}

Var mul(const Var& a, const Var& b) {
  Tensor out = t_binary(OXI_BINARY_MUL, a.value(), b.value());
  Tensor av = a.value(), bv = b.value();
  return Var::op(out, "mul", {a, b}, [av, bv](const Tensor& g, const std::vector<bool>& need) -> Grads {
    Grads r(2);
    if (need[0]) r[0] = bin(OXI_BINARY_MUL, g, bv);
    if (need[1]) r[1] = bin(OXI_BINARY_MUL, g, av);
    return r;
  });
}

Var div(const Var& a, const Var& b) {
  Tensor out = t_binary(OXI_BINARY_DIV, a.value(), b.value());
  Tensor av = a.value(), bv = b.value();
  return Var::op(out, "div", {a, b}, [av, bv](const Tensor& g, const std::vector<bool>& need) -> Grads {
    Grads r(2);
    if (need[0]) r[0] = bin(OXI_BINARY_DIV, g, bv);
    if (need[1]) {
      Tensor b2 = bin(OXI_BINARY_MUL, bv, bv);
      r[1] = un(OXI_UNARY_NEG, bin(OXI_BINARY_DIV, bin(OXI_BINARY_MUL, g, av), b2));
    }
    return r;
  });
}

Var pow(const Var& a, const Var& b) {
  Tensor out = t_binary(OXI_BINARY_POW, a.value(), b.value());
  Tensor av = a.value(), bv = b.value();
  return Var::op(out, "pow", {a, b}, [av, bv](const Tensor& g, const std::vector<bool>& need) -> Grads {
    Grads r(2);
    if (need[0]) {
      Tensor bm1 = bin(OXI_BINARY_ADD, bv, t_scalar_full({}, -1.0f, bv.dev()));
      Tensor apow = bin(OXI_BINARY_POW, av, bm1);
      r[0] = bin(OXI_BINARY_MUL, bin(OXI_BINARY_MUL, g, bv), apow);
    }
    if (need[1]) {
      Tensor o = bin(OXI_BINARY_POW, av, bv);
      r[1] = bin(OXI_BINARY_MUL, bin(OXI_BINARY_MUL, g, o), un(OXI_UNARY_LOG, av));
    }
    return r;
  });
}

// ---- unary (ops.rs:126-268) --------------------------------------------------------

namespace {
// unary_generic: gx = g * dfdx(x), dfdx recomputed from the saved input
Var unary_generic(const Var& x, int fwd_op, const char* name, std::function<Tensor(const Tensor&)> dfdx) {
  Tensor out = t_unary(fwd_op, x.value());
  Tensor xv = x.value();
  return Var::op(out, name, {x}, [xv, dfdx](const Tensor& g, const std::vector<bool>& need) -> Grads {
    if (!need[0]) return {std::nullopt};
    return {bin(OXI_BINARY_MUL, g, dfdx(xv))};
  });
}
}  // namespace

Var neg(const Var& x) {
  Tensor out = t_unary(OXI_UNARY_NEG, x.value());
  return Var::op(out, "neg", {x}, [](const Tensor& g, const std::vector<bool>& need) -> Grads {
    if (!need[0]) return {std::nullopt};
    return {un(OXI_UNARY_NEG, g)};
  });
}

Var abs(const Var& x) {
  return unary_generic(x, OXI_UNARY_ABS, "abs", [](const Tensor& t) { return un(OXI_UNARY_SIGN, t); });
}

Var exp(const Var& x) {
  return unary_generic(x, OXI_UNARY_EXP, "exp", [](const Tensor& t) { return un(OXI_UNARY_EXP, t); });
}

Var log(const Var& x) {
  return unary_generic(x, OXI_UNARY_LOG, "log",
                       [](const Tensor& t) { return bin(OXI_BINARY_DIV, ones_of(t), t); });
}

Var sqrt(const Var& x) {
  return unary_generic(x, OXI_UNARY_SQRT, "sqrt", [](const Tensor& t) {
    Tensor denom = bin(OXI_BINARY_MUL, un(OXI_UNARY_SQRT, t), t_scalar_full(t.shape, 2.0f, t.dev()));
    return bin(OXI_BINARY_DIV, ones_of(t), denom);
  });
}

Var tanh(const Var& x) {
  return unary_generic(x, OXI_UNARY_TANH, "tanh", [](const Tensor& t) {
    Tensor th = un(OXI_UNARY_TANH, t);
    return bin(OXI_BINARY_SUB, ones_of(t), bin(OXI_BINARY_MUL, th, th));
  });
}

Var sigmoid(const Var& x) {
  return unary_generic(x, OXI_UNARY_SIGMOID, "sigmoid", [](const Tensor& t) {
    Tensor s = un(OXI_UNARY_SIGMOID, t);
    return bin(OXI_BINARY_MUL, s, bin(OXI_BINARY_SUB, ones_of(t), s));
  });
}

Var relu(const Var& x) {  // ops.rs:254-268: grad mask x > 0
  Tensor out = t_unary(OXI_UNARY_RELU, x.value());
  Tensor mask = t_binary(OXI_CMP_GT, x.value(), t_scalar_full(x.value().shape, 0.0f, x.value().dev()));
  return Var::op(out, "relu", {x}, [mask](const Tensor& g, const std::vector<bool>& need) -> Grads {
    if (!need[0]) return {std::nullopt};
    return {bin(OXI_BINARY_MUL, g, mask)};
  });
}

// ---- reductions (ops.rs:327-388, 679-737) ---------------------------------------------

namespace {
// normalize_reduce_grad + expand_to: the upstream grad as a view of x's shape.
Tensor expand_grad(const Tensor& g, const Shape& x_shape, int dim) {
  if (g.shape == x_shape) return g;
  std::vector<int64_t> padded(g.shape.begin(), g.shape.end());
  if (g.shape.size() + 1 == x_shape.size()) padded.insert(padded.begin() + std::min<size_t>(dim, padded.size()), 1);
  Tensor r = t_reshape(g, padded);
  std::vector<int64_t> full(x_shape.size(), 1);
  const size_t tail = x_shape.size() - r.shape.size();
  for (size_t i = tail; i < x_shape.size(); ++i) full[i] = r.shape[i - tail];
  return t_broadcast_to(t_reshape(r, full), x_shape);
}
}  // namespace

Var reduce(const Var& x, Reduce kind, int64_t dim, bool keepdim) {
  Tensor out = t_reduce(kind, x.value(), dim, keepdim);
  const int d = normalize_dim(dim, x.value().ndim());
  const Shape xs = x.value().shape;
  Tensor xv = x.value();
  switch (kind) {
    case Reduce::Sum:
      return Var::op(out, "sum", {x}, [xs, d](const Tensor& g, const std::vector<bool>& need) -> Grads {
        if (!need[0]) return {std::nullopt};
        return {expand_grad(g, xs, d)};
      });
    case Reduce::Mean: {
      const float n = (float)xs[d];
      return Var::op(out, "mean", {x}, [xs, d, n](const Tensor& g, const std::vector<bool>& need) -> Grads {
        if (!need[0]) return {std::nullopt};
        Tensor up = expand_grad(g, xs, d);
        return {t_binary(OXI_BINARY_MUL, up, t_scalar_full(xs, 1.0f / n, up.dev()))};
      });
    }
    case Reduce::Max:
    case Reduce::Min: {
      // winners captured at forward; the grad goes to the single first winner
      Tensor arg = t_reduce(kind == Reduce::Max ? Reduce::ArgMax : Reduce::ArgMin, xv, d, true);
      return Var::op(out, "maxmin", {x}, [xs, d, arg](const Tensor& g, const std::vector<bool>& need) -> Grads {
        if (!need[0]) return {std::nullopt};
        Tensor up = expand_grad(g, xs, d);
        std::vector<float> pos((size_t)xs[d]);
        for (int64_t k = 0; k < xs[d]; ++k) pos[(size_t)k] = (float)k;
        Shape ps(xs.size(), 1);
        ps[d] = xs[d];
        Tensor positions = t_from_host(pos.data(), ps, Dev::Hip);
        Tensor mask = t_binary(OXI_CMP_EQ, t_broadcast_to(positions, xs), t_broadcast_to(arg, xs));
        return {t_binary(OXI_BINARY_MUL, mask, up)};
      });
    }
    case Reduce::Norm:
      return Var::op(out, "norm", {x}, [xs, d, xv](const Tensor& g, const std::vector<bool>& need) -> Grads {
        if (!need[0]) return {std::nullopt};
        Tensor up = expand_grad(g, xs, d);
        Tensor n = t_reduce(Reduce::Norm, xv, d, true);
        Tensor safe = t_binary(OXI_BINARY_ADD, n, t_scalar_full(n.shape, 1e-12f, n.dev()));
        Tensor ratio = t_binary(OXI_BINARY_DIV, xv, safe);
        return {t_binary(OXI_BINARY_MUL, up, ratio)};
      });
    default:
      err_notimpl("argmax/argmin are integer outputs and have no gradient");
  }
}

// ---- views (ops.rs:396-488) -------------------------------------------------------

Var reshape(const Var& x, const std::vector<int64_t>& shape) {
  Tensor out = t_reshape(x.value(), shape);
  const Shape orig = x.value().shape;
  return Var::op(out, "reshape", {x}, [orig](const Tensor& g, const std::vector<bool>& need) -> Grads {
    if (!need[0]) return {std::nullopt};
    return {t_reshape(g, orig)};
  });
}

Var permute(const Var& x, const std::vector<int64_t>& order) {
  Tensor out = t_permute(x.value(), order);
  std::vector<int64_t> inv(order.size());
  for (size_t i = 0; i < order.size(); ++i) inv[(size_t)normalize_dim(order[i], (int)order.size())] = (int64_t)i;
  Var v = Var::op(out, "permute", {x}, [inv](const Tensor& g, const std::vector<bool>& need) -> Grads {
    if (!need[0]) return {std::nullopt};
    return {t_permute(g, inv)};
  });
  if (v.node->op)
    for (int64_t o : order) v.node->perm.push_back((int64_t)normalize_dim(o, (int)order.size()));
  return v;
}

Var transpose(const Var& x) {
  Tensor out = t_transpose(x.value());
  Var v = Var::op(out, "transpose", {x}, [](const Tensor& g, const std::vector<bool>& need) -> Grads {
    if (!need[0]) return {std::nullopt};
    return {t_transpose(g)};
  });
  if (v.node->op) v.node->perm = {1, 0};
  return v;
}

Var broadcast_to(const Var& x, const Shape& shape) {
  Tensor out = t_broadcast_to(x.value(), shape);
  const Shape xs = x.value().shape;
  return Var::op(out, "broadcast_to", {x}, [xs](const Tensor& g, const std::vector<bool>& need) -> Grads {
    if (!need[0]) return {std::nullopt};
    return {unbroadcast(g, xs)};
  });
}

// The reference's narrow_dim0 (ops.rs:428-442) pads the gradient with zero
// rows; here the window of a zero tensor is written through a strided view.
Var narrow(const Var& x, int64_t dim, int64_t lo, int64_t hi, int64_t by) {
  Tensor out = t_narrow(x.value(), dim, lo, hi, by);
  const Shape xs = x.value().shape;
  return Var::op(out, "narrow", {x}, [xs, dim, lo, hi, by](const Tensor& g, const std::vector<bool>& need) -> Grads {
    if (!need[0]) return {std::nullopt};
    Tensor z = t_zeros(xs, g.dev());
    t_copy_into(t_narrow(z, dim, lo, hi, by), g);
    return {z};
  });
}

// ---- index_select (ops.rs:498-517, 741-769) -----------------------------------------

// The VJP's id sort is queued at forward time on the library's second stream
// (oxi_index_select_bwd_plan), where it overlaps the rest of the forward; the
// backward only waits for it and runs the segment sums.
Var index_select(const Var& x, int64_t dim, const std::vector<int64_t>& indices) {
  if (!is_grad_enabled() || !x.requires_grad()) return Var::leaf(t_index_select(x.value(), dim, indices), false);
  if (x.value().ndim() == 0) err_invalid("dim " + std::to_string(dim) + " out of range for 0-D tensor");
  const int d = normalize_dim(dim, x.value().ndim());
  const Shape xs = x.value().shape;
  auto ids = device_i64(resolve_indices(indices, xs[d], d));
  const int64_t n = (int64_t)indices.size();
  // the sort is queued first so that it overlaps the gather itself
  void* raw = nullptr;
  hip_check(oxi_index_select_bwd_plan(static_cast<const int64_t*>(ids->ptr), n, xs[d], &raw));
  std::shared_ptr<void> plan(raw, [ids](void* p) { (void)oxi_index_select_bwd_plan_free(p); });
  Tensor out = t_index_select_dev(x.value(), d, ids, n);
  return Var::op(out, "index_select", {x}, [xs, d, plan](const Tensor& g, const std::vector<bool>& need) -> Grads {
    if (!need[0]) return {std::nullopt};
    Tensor gc = t_contiguous(g);
    int64_t outer = 1, inner = 1;
    for (int i = 0; i < d; ++i) outer *= xs[i];
    for (size_t i = d + 1; i < xs.size(); ++i) inner *= xs[i];
    Tensor grad = Tensor::empty(xs, Dev::Hip);
    hip_check(oxi_index_select_bwd_apply(plan.get(), gc.data(), outer, inner, grad.data()));
    return {grad};
  });
}

// aops::scatter_dim0 (crates/oxi-autograd/src/ops.rs:531-600): the written
// rows of base get no gradient, the last writer of each row gets that row's.
Var scatter_dim0(const Var& base, const std::vector<int64_t>& indices, const Var& values) {
  Tensor out = t_scatter_dim0(base.value(), indices, values.value());
  const Shape bs = base.value().shape;
  const Shape vs = values.value().shape;
  const int64_t rows = bs[0];
  int64_t inner = 1;
  for (size_t d = 1; d < bs.size(); ++d) inner *= bs[d];
  auto ids = device_i64(resolve_indices(indices, rows, 0));
  const int64_t n = (int64_t)indices.size();
  return Var::op(out, "scatter_dim0", {base, values},
                 [bs, vs, rows, inner, ids, n](const Tensor& g, const std::vector<bool>& need) -> Grads {
                   std::optional<Tensor> gb, gv;
                   if (need[0]) gb = Tensor::empty(bs, Dev::Hip);
                   if (need[1]) gv = Tensor::empty(vs, Dev::Hip);
                   if (gb || gv) {
                     Tensor gc = t_contiguous(g);
                     hip_check(oxi_scatter_rows_bwd(gc.data(), rows, inner, static_cast<const int64_t*>(ids->ptr), n,
                                                    gb ? gb->data() : nullptr, gv ? gv->data() : nullptr));
                   }
                   return {gb, gv};
                 });
}

// aops::masked_select (crates/oxi-autograd/src/ops.rs:609-667): each pick's
// gradient goes back to its x element, accumulating over broadcast points.
// The VJP keeps the forward's selection record (one bit per grid point)
// instead of x and the mask.
Var masked_select(const Var& x, const Var& mask) {
  const bool record = is_grad_enabled() && x.requires_grad();
  std::shared_ptr<Storage> rec;
  Tensor out = t_masked_select(x.value(), mask.value(), record ? &rec : nullptr);
  const Shape xshape = x.value().shape;
  const Shape grid = broadcast_shapes(xshape, mask.value().shape);
  const int64_t count = out.numel();
  return Var::op(out, "masked_select", {x},
                 [rec, xshape, grid, count](const Tensor& g, const std::vector<bool>& need) -> Grads {
                   if (!need[0]) return {std::nullopt};
                   if (!rec) err_other("masked_select: the forward kept no selection record");
                   // row-major strides of x's own shape on the grid, 0 where x
                   // broadcasts (a missing or size-1 dim): x_flat_str, ops.rs:628-634
                   const Shape rm = row_major_strides(xshape);
                   const size_t lead = grid.size() - xshape.size();
                   Shape gxs(grid.size(), 0);
                   for (size_t d = lead; d < grid.size(); ++d)
                     if (xshape[d - lead] != 1) gxs[d] = rm[d - lead];
                   Tensor gc = t_contiguous(g);
                   Tensor gx = Tensor::empty(xshape, Dev::Hip);
                   hip_check(oxi_masked_select_bwd(rec->ptr, grid.data(), (int)grid.size(), gc.data(), count,
                                                   gx.data(), gxs.data(), gx.numel()));
                   return {gx};
                 });
}

Var embedding(const std::vector<int64_t>& indices, const Var& weight) {
  return index_select(weight, 0, indices);
}

// ---- fused norms (functional.py:227-240) ----------------------------------------------

NormVjp norm_vjp_mode() {
  const char* e = std::getenv("OXI_NORM_VJP");
  if (!e || !*e || std::strcmp(e, "ref") == 0) return NormVjp::Ref;
  if (std::strcmp(e, "exact") == 0) return NormVjp::Exact;
  err_invalid(std::string("OXI_NORM_VJP must be \"ref\" or \"exact\", got \"") + e + "\"");
}

namespace {
int64_t last_dim(const Tensor& x, const char* what) {
  if (x.ndim() == 0) err_invalid(std::string(what) + " needs at least one dim");
  return x.shape.back();
}
void check_param(const Tensor& p, int64_t H, const char* what) {
  if (p.ndim() != 1 || p.shape[0] != H) err_shape(fmt_shape(p.shape), fmt_shape({H}));
  (void)what;
}
}  // namespace

Var rms_norm(const Var& x, const Var& w, float eps, NormVjp mode) {
  const int64_t H = last_dim(x.value(), "rms_norm");
  check_param(w.value(), H, "weight");
  Tensor xc = t_contiguous(x.value());
  Tensor wc = t_contiguous(w.value());
  const int64_t rows = H ? xc.numel() / H : 0;
  Tensor y = Tensor::empty(xc.shape, Dev::Hip);
  Tensor rstd = Tensor::empty({rows}, Dev::Hip);
  hip_check(oxi_rms_norm_fwd(xc.data(), wc.data(), y.data(), rstd.data(), rows, H, eps));
  auto saved = std::make_shared<NormSaved>();
  saved->x = xc;
  saved->w = wc;
  saved->has_w = true;
  saved->rstd = rstd;
  saved->rows = rows;
  saved->H = H;
  saved->mode = (int)mode;
  saved->wi = 1;
  Var v = Var::op(y, "rms_norm", {x, w}, [xc, wc, rstd, rows, H, mode](const Tensor& g, const std::vector<bool>& need) {
    Grads r(2);
    Tensor gc = t_contiguous(g);
    Tensor dx, dw;
    if (need[0]) dx = Tensor::empty(xc.shape, Dev::Hip);
    if (need[1]) dw = Tensor::empty({H}, Dev::Hip);
    if (!need[0] && !need[1]) return r;
    hip_check(oxi_rms_norm_bwd(xc.data(), wc.data(), rstd.data(), gc.data(), need[0] ? dx.data() : nullptr,
                               need[1] ? dw.data() : nullptr, rows, H, (int)mode));
    if (need[0]) r[0] = dx;
    if (need[1]) r[1] = dw;
    return r;
  });
  if (v.node->op) v.node->norm = std::move(saved);
  return v;
}

Var layer_norm(const Var& x, const std::optional<Var>& w, const std::optional<Var>& b, float eps, NormVjp mode) {
  const int64_t H = last_dim(x.value(), "layer_norm");
  if (w) check_param(w->value(), H, "weight");
  if (b) check_param(b->value(), H, "bias");
  Tensor xc = t_contiguous(x.value());
  Tensor wc = w ? t_contiguous(w->value()) : Tensor();
  Tensor bc = b ? t_contiguous(b->value()) : Tensor();
  const int64_t rows = H ? xc.numel() / H : 0;
  Tensor y = Tensor::empty(xc.shape, Dev::Hip);
  Tensor mean = Tensor::empty({rows}, Dev::Hip);
  Tensor rstd = Tensor::empty({rows}, Dev::Hip);
  hip_check(oxi_layer_norm_fwd(xc.data(), w ? wc.data() : nullptr, b ? bc.data() : nullptr, y.data(), mean.data(),
                               rstd.data(), rows, H, eps));
  std::vector<Var> inputs{x};
  const int wi = w ? (int)inputs.size() : -1;
  if (w) inputs.push_back(*w);
  const int bi = b ? (int)inputs.size() : -1;
  if (b) inputs.push_back(*b);
  const bool has_w = (bool)w;
  auto saved = std::make_shared<NormSaved>();
  saved->ln = true;
  saved->x = xc;
  saved->w = wc;
  saved->b = bc;
  saved->has_w = has_w;
  saved->has_b = (bool)b;
  saved->mean = mean;
  saved->rstd = rstd;
  saved->rows = rows;
  saved->H = H;
  saved->mode = (int)mode;
  saved->wi = wi;
  saved->bi = bi;
  Var v = Var::op(y, "layer_norm", inputs,
                 [xc, wc, mean, rstd, rows, H, mode, wi, bi, has_w](const Tensor& g, const std::vector<bool>& need) {
                   Grads r(need.size());
                   const bool ndx = need[0], ndw = wi >= 0 && need[wi], ndb = bi >= 0 && need[bi];
                   if (!ndx && !ndw && !ndb) return r;
                   Tensor gc = t_contiguous(g);
                   Tensor dx = ndx ? Tensor::empty(xc.shape, Dev::Hip) : Tensor();
                   Tensor dw = ndw ? Tensor::empty({H}, Dev::Hip) : Tensor();
                   Tensor db = ndb ? Tensor::empty({H}, Dev::Hip) : Tensor();
                   hip_check(oxi_layer_norm_bwd(xc.data(), has_w ? wc.data() : nullptr, mean.data(), rstd.data(),
                                                gc.data(), ndx ? dx.data() : nullptr, ndw ? dw.data() : nullptr,
                                                ndb ? db.data() : nullptr, rows, H, (int)mode));
                   if (ndx) r[0] = dx;
                   if (ndw) r[wi] = dw;
                   if (ndb) r[bi] = db;
                   return r;
                 });
  if (v.node->op) v.node->norm = std::move(saved);
  return v;
}

bool norm_vjp_fused(const NormSaved& s, int act, const Tensor& g, const std::vector<bool>& need, Tensor* dy,
                    Grads& grads, int64_t lead, Tensor* lsum) {
  grads.assign(need.size(), std::nullopt);
  const bool ndx = need[0] || lsum, ndw = s.wi >= 0 && need[s.wi], ndb = s.bi >= 0 && need[s.bi];
  Tensor gc = t_contiguous(g.shape == s.x.shape ? g : t_broadcast_to(g, s.x.shape));
  const bool ndy = act >= 0 && dy;  // the activation's input gradient, when the caller keeps it
  Tensor d = ndy ? Tensor::empty(s.x.shape, Dev::Hip) : Tensor();
  Tensor dx = ndx ? Tensor::empty(s.x.shape, Dev::Hip) : Tensor();
  Tensor dw = ndw ? Tensor::empty({s.H}, Dev::Hip) : Tensor();
  Tensor db = ndb ? Tensor::empty({s.H}, Dev::Hip) : Tensor();
  Tensor ls = lsum ? Tensor::empty({s.rows / lead, s.H}, Dev::Hip) : Tensor();
  const float* w = s.has_w ? s.w.data() : nullptr;
  const float* b = s.has_b ? s.b.data() : nullptr;
  float* dp = ndy ? d.data() : nullptr;
  float* dxp = ndx ? dx.data() : nullptr;
  float* dwp = ndw ? dw.data() : nullptr;
  float* dbp = ndb ? db.data() : nullptr;
  int rc;
  if (lsum)
    rc = s.ln ? oxi_layer_norm_bwd_lead_sum(s.x.data(), w, b, s.mean.data(), s.rstd.data(), gc.data(), act, dp, dxp,
                                            dwp, dbp, ls.data(), lead, s.rows, s.H, s.mode)
              : oxi_rms_norm_bwd_lead_sum(s.x.data(), w, s.rstd.data(), gc.data(), act, dp, dxp, dwp, ls.data(),
                                          lead, s.rows, s.H, s.mode);
  else if (act >= 0)
    rc = s.ln ? oxi_layer_norm_act_bwd(s.x.data(), w, b, s.mean.data(), s.rstd.data(), gc.data(), act, dp, dxp, dwp,
                                       dbp, s.rows, s.H, s.mode)
              : oxi_rms_norm_act_bwd(s.x.data(), w, s.rstd.data(), gc.data(), act, dp, dxp, dwp, s.rows, s.H,
                                     s.mode);
  else
    return false;
  if (rc == OXI_NOT_IMPLEMENTED) return false;
  hip_check(rc);
  if (ndy) *dy = d;
  if (lsum) *lsum = ls;
  if (need[0]) grads[0] = dx;
  if (ndw) grads[s.wi] = dw;
  if (ndb) grads[s.bi] = db;
  return true;
}

// ---- fused activations (functional.py:194-204) ----------------------------------------

Var gelu(const Var& x, int approximate) {
  const Tensor& xv = x.value();
  require_hip(xv, "gelu");
  Tensor y = Tensor::empty(xv.shape, Dev::Hip);
  hip_check(oxi_gelu_fwd(xv.data(), xv.strides.data(), y.data(), y.strides.data(), xv.shape.data(), xv.ndim(),
                         approximate));
  Tensor xs = xv;
  Var v = Var::op(y, "gelu", {x}, [xs, approximate](const Tensor& g, const std::vector<bool>& need) -> Grads {
    if (!need[0]) return {std::nullopt};
    Tensor gb = g.shape == xs.shape ? g : t_broadcast_to(g, xs.shape);
    Tensor dx = Tensor::empty(xs.shape, Dev::Hip);
    dx.strides = result_strides(xs.shape, {&xs, &gb});
    hip_check(oxi_gelu_bwd(xs.data(), xs.strides.data(), gb.data(), gb.strides.data(), dx.data(), dx.strides.data(),
                           xs.shape.data(), xs.ndim(), approximate));
    return {dx};
  });
  if (v.node->op) v.node->act = approximate == OXI_GELU_ERF ? OXI_ACT_GELU_ERF : OXI_ACT_GELU_TANH;
  return v;
}

Var silu(const Var& x) {
  const Tensor& xv = x.value();
  require_hip(xv, "silu");
  Tensor y = Tensor::empty(xv.shape, Dev::Hip);
  hip_check(oxi_silu_fwd(xv.data(), xv.strides.data(), y.data(), y.strides.data(), xv.shape.data(), xv.ndim()));
  Tensor xs = xv;
  Var v = Var::op(y, "silu", {x}, [xs](const Tensor& g, const std::vector<bool>& need) -> Grads {
    if (!need[0]) return {std::nullopt};
    Tensor gb = g.shape == xs.shape ? g : t_broadcast_to(g, xs.shape);
    Tensor dx = Tensor::empty(xs.shape, Dev::Hip);
    dx.strides = result_strides(xs.shape, {&xs, &gb});
    hip_check(oxi_silu_bwd(xs.data(), xs.strides.data(), gb.data(), gb.strides.data(), dx.data(), dx.strides.data(),
                           xs.shape.data(), xs.ndim()));
    return {dx};
  });
  if (v.node->op) v.node->act = OXI_ACT_SILU;
  return v;
}

// ---- softmax family (functional.py:211-222) ---------------------------------------------

Var softmax(const Var& x, int64_t dim, bool log) {
  const Tensor& xv = x.value();
  if (xv.ndim() == 0) err_invalid("dim " + std::to_string(dim) + " out of range for 0-D tensor");
  const int d = normalize_dim(dim, xv.ndim());
  if (xv.shape[d] == 0) err_invalid("cannot compute max/min over a zero-length dim");
  Tensor xc = t_contiguous(xv);
  int64_t outer = 1, inner = 1;
  for (int i = 0; i < d; ++i) outer *= xv.shape[i];
  for (int i = d + 1; i < xv.ndim(); ++i) inner *= xv.shape[i];
  const int64_t len = xv.shape[d];
  Tensor y = Tensor::empty(xv.shape, Dev::Hip);
  hip_check(log ? oxi_log_softmax_fwd(xc.data(), y.data(), outer, len, inner)
                : oxi_softmax_fwd(xc.data(), y.data(), outer, len, inner));
  Var v = Var::op(y, log ? "log_softmax" : "softmax", {x},
                  [y, outer, len, inner, log](const Tensor& g, const std::vector<bool>& need) -> Grads {
                    if (!need[0]) return {std::nullopt};
                    Tensor gc = t_contiguous(g.shape == y.shape ? g : t_broadcast_to(g, y.shape));
                    Tensor dx = Tensor::empty(y.shape, Dev::Hip);
                    hip_check(log ? oxi_log_softmax_bwd(y.data(), gc.data(), dx.data(), outer, len, inner)
                                  : oxi_softmax_bwd(y.data(), gc.data(), dx.data(), outer, len, inner));
                    return {dx};
                  });
  // over the last dim a norm VJP can absorb it
  if (v.node->op && inner == 1) v.node->act = log ? OXI_ACT_LOG_SOFTMAX : OXI_ACT_SOFTMAX;
  return v;
}

// ---- cross entropy (functional.py:277-293), targets already resolved ------------------------

Var cross_entropy(const Var& logits, const std::vector<int64_t>& targets) {
  const Tensor& lv = logits.value();
  if (lv.ndim() != 2) err_invalid("cross_entropy expects (batch, classes) logits, got " + fmt_shape(lv.shape));
  const int64_t n = lv.shape[0], c = lv.shape[1];
  if ((int64_t)targets.size() != n)
    err_invalid(std::to_string(targets.size()) + " targets for batch of " + std::to_string(n));
  for (int64_t t : targets)
    if (t < 0 || t >= c)
      err_oob("index " + std::to_string(t) + " is out of bounds for axis 1 with size " + std::to_string(c));
  require_hip(lv, "cross_entropy");
  Tensor lc = t_contiguous(lv);
  auto tg = device_i64(targets);
  const int64_t* tp = static_cast<const int64_t*>(tg->ptr);
  Tensor loss = Tensor::empty({}, Dev::Hip);
  Tensor lse = Tensor::empty({n}, Dev::Hip);
  // With a gradient to come, the forward pass also forms the gradient for an
  // upstream 1 (loss.backward()'s seed) from the logits it holds: the first
  // backward seeded so takes it as is; any other upstream, or a second
  // backward, runs the backward kernel. That gradient is an n x c tensor held
  // until the backward: a loop that scales the loss first, or never calls
  // backward, pays its write and memory for nothing, and turns it off with
  // OXI_CE_ONE_PASS=0 (or set_ce_one_pass(False)).
  std::optional<Tensor> unit;
  if (logits.requires_grad() && is_grad_enabled() && ce_one_pass()) {
    Tensor d = Tensor::empty({n, c}, Dev::Hip);
    const int rc = oxi_cross_entropy_fwd_grad(lc.data(), tp, loss.data(), lse.data(), d.data(), n, c);
    if (rc == OXI_OK) unit = d;
    else if (rc != OXI_NOT_IMPLEMENTED) hip_check(rc);
  }
  if (!unit) hip_check(oxi_cross_entropy_fwd(lc.data(), tp, loss.data(), lse.data(), n, c));
  auto fresh = std::make_shared<std::atomic<bool>>(unit.has_value());
  return Var::op(loss, "cross_entropy", {logits},
                 [lc, tg, lse, n, c, unit, fresh](const Tensor& g, const std::vector<bool>& need) -> Grads {
                   if (!need[0]) return {std::nullopt};
                   if (is_implicit_seed(g) && fresh->exchange(false)) return {*unit};
                   Tensor gs = t_contiguous(g);
                   Tensor d = Tensor::empty({n, c}, Dev::Hip);
                   hip_check(oxi_cross_entropy_bwd(lc.data(), static_cast<const int64_t*>(tg->ptr), lse.data(),
                                                   gs.data(), d.data(), n, c));
                   return {d};
                 });
}

}  // namespace aops
}  // namespace oxt
