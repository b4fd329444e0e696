// Autograd graph: restates crates/oxi-autograd/src/graph.rs (Var/Node, the
// thread-local grad mode, accumulate_grad, unbroadcast, topo_order and
// backward_ext) over device tensors.
#include <atomic>
#include <cstdlib>
#include <cstring>
#include <unordered_map>
#include <unordered_set>

#include "host.h"

namespace oxt {

namespace {
thread_local bool g_grad_enabled = true;  // graph.rs:30-48
}

bool is_grad_enabled() { return g_grad_enabled; }
bool set_grad_enabled(bool on) {
  const bool prev = g_grad_enabled;
  g_grad_enabled = on;
  return prev;
}

Var Var::leaf(Tensor value, bool requires_grad) {
  Var v;
  v.node = std::make_shared<Node>();
  v.node->value = std::move(value);
  v.node->requires_grad = requires_grad;
  return v;
}

// graph.rs:157-177: under no_grad the result is a detached leaf.
Var Var::op(Tensor value, const char* name, std::vector<Var> inputs, Vjp vjp) {
  if (!is_grad_enabled()) return leaf(std::move(value), false);
  bool rg = false;
  for (const Var& i : inputs) rg = rg || i.requires_grad();
  Var v;
  v.node = std::make_shared<Node>();
  v.node->value = std::move(value);
  v.node->op = name;
  v.node->inputs = std::move(inputs);
  v.node->vjp = std::move(vjp);
  v.node->requires_grad = rg;
  return v;
}

namespace {
// The node's gradient, forming a deferred one first (outside the node's lock:
// forming it launches kernels).
std::optional<Tensor> read_grad(Node& nd) {
  std::shared_ptr<DeferredGrad> d;
  {
    std::lock_guard<std::mutex> lk(nd.mu);
    if (nd.grad || !nd.dgrad) return nd.grad;
    d = nd.dgrad;
  }
  Tensor g = d->get();
  std::lock_guard<std::mutex> lk(nd.mu);
  if (nd.dgrad == d) {
    nd.grad = g;
    nd.dgrad.reset();
  }
  return nd.grad;
}
}  // namespace

std::optional<Tensor> Var::grad() const { return read_grad(*node); }

void Var::set_grad(const Tensor& g) const {  // graph.rs:208-217
  if (g.shape != node->value.shape) err_shape(fmt_shape(g.shape), fmt_shape(node->value.shape));
  std::lock_guard<std::mutex> lk(node->mu);
  node->grad = g;
  node->dgrad.reset();
}

void Var::clear_grad() const {
  std::lock_guard<std::mutex> lk(node->mu);
  node->grad.reset();
  node->dgrad.reset();
}

void Var::zero_grad() const {  // graph.rs:229-233
  Tensor z = t_zeros(node->value.shape, node->value.dev());
  std::lock_guard<std::mutex> lk(node->mu);
  node->grad = z;
  node->dgrad.reset();
}

void Var::accumulate_grad(const Tensor& g) const {  // graph.rs:235-242
  (void)read_grad(*node);  // a deferred gradient is formed before anything is added to it
  std::lock_guard<std::mutex> lk(node->mu);
  if (!node->grad) node->grad = g;
  else node->grad = t_add(*node->grad, g);
}

// graph.rs:274-313
Tensor unbroadcast(const Tensor& g, const Shape& shape) {
  const Shape& gs = g.shape;
  if (gs.size() < shape.size()) err_shape(fmt_shape(gs), fmt_shape(shape));
  const size_t extra = gs.size() - shape.size();
  for (size_t i = 0; i < shape.size(); ++i) {
    const int64_t gi = gs[extra + i];
    if (gi != shape[i] && shape[i] != 1) err_shape(fmt_shape(gs), fmt_shape(shape));
  }
  Tensor t = g;
  for (size_t i = 0; i < extra; ++i) t = t_reduce(Reduce::Sum, t, (int64_t)i, true);
  for (size_t i = 0; i < shape.size(); ++i)
    if (shape[i] == 1 && t.shape[i] != 1) t = t_reduce(Reduce::Sum, t, (int64_t)i, true);
  if (t.shape != shape) t = t_reshape(t, shape);
  return t;
}

namespace {
// graph.rs:316-349: iterative DFS, post-order.
std::vector<Var> topo_order(const Var& root) {
  struct Frame {
    bool exit;
    Var v;
  };
  std::vector<Var> order;
  std::unordered_set<const Node*> visited;
  std::vector<Frame> stack{{false, root}};
  while (!stack.empty()) {
    Frame f = stack.back();
    stack.pop_back();
    if (!f.exit) {
      if (!visited.insert(f.v.node.get()).second) continue;
      stack.push_back({true, f.v});
      const std::vector<Var> inputs = f.v.node->inputs;
      for (const Var& in : inputs)
        if (!visited.count(in.node.get())) stack.push_back({false, in});
    } else {
      order.push_back(f.v);
    }
  }
  return order;
}
}  // namespace

namespace {
// -1: follow OXI_FUSE_NORM_ACT; 0 / 1: set by set_fuse_norm_act
std::atomic<int> g_fuse_override{-1};
std::atomic<uint64_t> g_fused_passes{0};

// Takes the node's VJP (a copy when the graph is retained), raising the
// reference's error when an earlier pass consumed it (graph.rs:405-420).
Vjp take_vjp(Node& nd, bool retain_graph) {
  std::lock_guard<std::mutex> lk(nd.mu);
  if (!nd.vjp) {
    if (retain_graph) err_invalid("internal: op node reached in backward without a VJP");
    err_invalid(
        "trying to backward through the graph a second time (or along an already freed path): pass "
        "retain_graph=True on the first backward call");
  }
  if (retain_graph) return *nd.vjp;
  Vjp f = std::move(*nd.vjp);
  nd.vjp.reset();
  return f;
}
}  // namespace

bool fuse_norm_act() {
  const int o = g_fuse_override.load();
  if (o >= 0) return o == 1;
  const char* e = std::getenv("OXI_FUSE_NORM_ACT");
  return !(e && std::strcmp(e, "0") == 0);
}

uint64_t fused_norm_act_passes() { return g_fused_passes.load(); }

namespace {
// -1: follow OXI_CE_ONE_PASS; 0 / 1: set by set_ce_one_pass
std::atomic<int> g_ce_override{-1};
}  // namespace

bool ce_one_pass() {
  const int o = g_ce_override.load();
  if (o >= 0) return o == 1;
  const char* e = std::getenv("OXI_CE_ONE_PASS");
  return !(e && std::strcmp(e, "0") == 0);
}

bool set_ce_one_pass(bool on) {
  const bool prev = ce_one_pass();
  g_ce_override.store(on ? 1 : 0);
  return prev;
}

bool set_fuse_norm_act(bool on) {
  const bool prev = fuse_norm_act();
  g_fuse_override.store(on ? 1 : 0);
  return prev;
}

namespace {
bool has_vjp(Node* nd) {
  std::lock_guard<std::mutex> lk(nd->mu);
  return (bool)nd->vjp;
}

// An add node r = p + q feeding a norm whose input it is, where q is
// broadcast over the leading dim only ((1, ...) against r's (lead, ...)): the
// norm pass can also form q's gradient, the sum of dx over that dim, which
// the add's VJP and unbroadcast would otherwise form in a pass of their own.
struct LeadSum {
  Node* add = nullptr;
  int qi = -1;
  int64_t lead = 0;
};

LeadSum lead_sum_of(Node* norm, const std::unordered_map<const Node*, int>& uses) {
  LeadSum ls;
  if (norm->inputs.empty()) return ls;
  Node* a = norm->inputs[0].node.get();
  auto u = uses.find(a);
  if (!a->op || std::strcmp(a->op, "add") != 0 || a->inputs.size() != 2 || u == uses.end() || u->second != 1 ||
      !has_vjp(a))
    return ls;
  const Shape& rs = a->value.shape;
  if (rs.size() < 2 || rs[0] < 2) return ls;
  for (int qi = 0; qi < 2; ++qi) {
    const Var& q = a->inputs[qi];
    const Shape& qs = q.value().shape;
    if (!q.requires_grad() || qs.size() != rs.size() || qs[0] != 1) continue;
    if (!std::equal(qs.begin() + 1, qs.end(), rs.begin() + 1)) continue;
    if (a->inputs[1 - qi].value().shape != rs) continue;
    ls.add = a;
    ls.qi = qi;
    ls.lead = rs[0];
    return ls;
  }
  return ls;
}

// The add node's gradients as its VJP and unbroadcast would give them: the
// norm's dx for the full operand, the leading-dim sum for the broadcast one.
std::vector<std::optional<Tensor>> add_grads(const LeadSum& ls, const std::optional<Tensor>& dx, const Tensor& dsum) {
  std::vector<std::optional<Tensor>> g(2);
  const Var& p = ls.add->inputs[1 - ls.qi];
  if (p.requires_grad()) g[1 - ls.qi] = dx;
  g[ls.qi] = t_reshape(dsum, ls.add->inputs[ls.qi].value().shape);
  return g;
}
}  // namespace

// graph.rs:373-438
//
// Additions to the reference's loop, each giving the same gradients with
// fewer passes over HBM (OXI_FUSE_NORM_ACT=0 turns them off):
// - when an activation node (gelu, silu, softmax, log_softmax) takes a norm
//   node's output, or, for the elementwise ones, a permuted view of it, and
//   that output feeds no other edge of this graph, the activation's VJP and
//   the norm's run as one pass (oxi_*_norm_act_bwd). The norm output's
//   gradient is still formed and stored (through the permute node, as its
//   VJP would pass it), and the norm's input gradients are held until the
//   loop reaches the norm node, so every accumulation happens in the
//   reference's order with the same values. The pass does not write the
//   norm output's gradient: that node (and the permute between, if any)
//   gets it deferred, formed on first read by the activation's own VJP (and
//   the permute's), so reading it gives the node-by-node values;
// - when the norm's input is r = p + q with q broadcast over the leading dim
//   (a positional table) and r feeds nothing else, the norm pass also forms
//   q's gradient (oxi_*_norm_bwd_lead_sum), held for the add node.
namespace {
thread_local const Storage* t_implicit_seed = nullptr;

struct SeedScope {
  const Storage* prev;
  explicit SeedScope(const Storage* st) : prev(t_implicit_seed) { t_implicit_seed = st; }
  ~SeedScope() { t_implicit_seed = prev; }
};
}  // namespace

bool is_implicit_seed(const Tensor& g) { return g.st && g.st.get() == t_implicit_seed; }

void backward(const Var& root, std::optional<Tensor> seed, bool retain_graph) {
  if (!root.requires_grad())
    err_invalid("element 0 of tensors does not require grad and does not have a grad_fn");
  Tensor s;
  if (seed) {
    s = *seed;
    if (s.shape != root.value().shape) s = t_broadcast_to(s, root.value().shape);
  } else if (root.value().numel() == 1) {
    s = t_ones_like(root.value());
  } else {
    err_invalid("grad can be implicitly created only for scalar outputs; pass a seed tensor");
  }
  SeedScope scope(seed ? nullptr : s.st.get());
  std::vector<Var> order = topo_order(root);
  for (Var& n : order)
    if (n.node->op) {
      std::lock_guard<std::mutex> lk(n.node->mu);
      n.node->grad.reset();
      n.node->dgrad.reset();
    }
  // edges into each node from the nodes of this graph
  const bool fuse = fuse_norm_act();
  std::unordered_map<const Node*, int> uses;
  if (fuse)
    for (const Var& n : order)
      for (const Var& in : n.node->inputs) ++uses[in.node.get()];
  std::unordered_map<const Node*, std::vector<std::optional<Tensor>>> held;  // gradients from a fused pass
  std::unordered_set<const Node*> through;  // permutes between a fused activation and its norm
  root.accumulate_grad(s);
  for (auto it = order.rbegin(); it != order.rend(); ++it) {
    Var& n = *it;
    if (!n.node->op) continue;
    std::vector<std::optional<Tensor>> grads;
    auto h = held.find(n.node.get());
    if (h != held.end()) {
      take_vjp(*n.node, retain_graph);  // computed by a fused pass
      grads = std::move(h->second);
      held.erase(h);
    } else if (through.count(n.node.get())) {
      // its gradient is deferred; the norm output's is this permute's VJP of it
      Vjp fv = take_vjp(*n.node, retain_graph);
      std::shared_ptr<DeferredGrad> dv;
      {
        std::lock_guard<std::mutex> lk(n.node->mu);
        dv = n.node->dgrad;
      }
      auto dn = std::make_shared<DeferredGrad>();
      dn->make = [fv, dv]() { return *fv(dv->get(), std::vector<bool>{true})[0]; };
      Node* nn = n.node->inputs[0].node.get();
      std::lock_guard<std::mutex> lk(nn->mu);
      nn->dgrad = std::move(dn);
      continue;
    } else {
      const std::optional<Tensor> up = read_grad(*n.node);
      if (!up) err_invalid("internal: node reached in backward without a gradient");
      std::vector<bool> needs;
      for (const Var& in : n.node->inputs) needs.push_back(in.requires_grad());
      Vjp f = take_vjp(*n.node, retain_graph);
      bool done = false;
      if (fuse && n.node->act >= 0 && n.node->inputs.size() == 1 && needs[0]) {
        // the norm node, directly or through one permute (elementwise activations only)
        Node* nn = n.node->inputs[0].node.get();
        Node* view = nullptr;
        if (!nn->norm && !nn->perm.empty() && n.node->act <= OXI_ACT_SILU && nn->inputs.size() == 1 &&
            uses[nn] == 1 && has_vjp(nn)) {
          view = nn;
          nn = nn->inputs[0].node.get();
        }
        if (nn->norm && uses[nn] == 1 && has_vjp(nn)) {
          std::vector<bool> nneeds;
          for (const Var& in : nn->inputs) nneeds.push_back(in.requires_grad());
          Tensor g = *up;
          if (view) {  // the activation's gradient in the norm output's layout
            std::vector<int64_t> inv(view->perm.size());
            for (size_t i = 0; i < inv.size(); ++i) inv[(size_t)view->perm[i]] = (int64_t)i;
            g = t_permute(g, inv);
          }
          LeadSum ls = lead_sum_of(nn, uses);
          Tensor dsum;
          std::vector<std::optional<Tensor>> ng;
          bool ok = ls.add && aops::norm_vjp_fused(*nn->norm, n.node->act, g, nneeds, nullptr, ng, ls.lead, &dsum);
          if (ok) held[ls.add] = add_grads(ls, ng[0], dsum);
          else ok = aops::norm_vjp_fused(*nn->norm, n.node->act, g, nneeds, nullptr, ng);
          if (ok) {
            // the activation's input gradient (its only edge) is formed on read
            auto d = std::make_shared<DeferredGrad>();
            d->make = [f, u = *up]() { return *f(u, std::vector<bool>{true})[0]; };
            Node* ain = n.node->inputs[0].node.get();
            {
              std::lock_guard<std::mutex> lk(ain->mu);
              ain->dgrad = std::move(d);
            }
            if (view) through.insert(view);
            held[nn] = std::move(ng);
            done = true;
            g_fused_passes.fetch_add(1);
          }
        }
      } else if (fuse && n.node->norm) {
        // a norm node whose VJP no activation pass took: fold the leading-dim
        // sum of a broadcast operand of its input into it
        LeadSum ls = lead_sum_of(n.node.get(), uses);
        Tensor dsum;
        if (ls.add && aops::norm_vjp_fused(*n.node->norm, OXI_ACT_NONE, *up, needs, nullptr, grads, ls.lead, &dsum)) {
          held[ls.add] = add_grads(ls, grads[0], dsum);
          done = true;
          g_fused_passes.fetch_add(1);
        }
      }
      if (!done) grads = f(*up, needs);
    }
    const std::vector<Var> inputs = n.node->inputs;
    for (size_t i = 0; i < inputs.size() && i < grads.size(); ++i) {
      if (!inputs[i].requires_grad() || !grads[i]) continue;
      inputs[i].accumulate_grad(unbroadcast(*grads[i], inputs[i].value().shape));
    }
  }
}

}  // namespace oxt
