// Autograd graph: restates crates/oxi-autograd/src/graph.rs (Var/Node, the
// thread-local grad mode, accumulate_grad, unbroadcast, topo_order and
// backward_ext) over device tensors.
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

std::optional<Tensor> Var::grad() const {
  std::lock_guard<std::mutex> lk(node->mu);
  return node->grad;
}

void Var::set_grad(const Tensor& g) const {  // graph.rs:208-217
  if (g.shape != node->value.shape) err_shape(fmt_shape(g.shape), fmt_shape(node->value.shape));
  std::lock_guard<std::mutex> lk(node->mu);
  node->grad = g;
}

void Var::zero_grad() const {  // graph.rs:229-233
  Tensor z = t_zeros(node->value.shape, node->value.dev());
  std::lock_guard<std::mutex> lk(node->mu);
  node->grad = z;
}

void Var::accumulate_grad(const Tensor& g) const {  // graph.rs:235-242
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

// graph.rs:373-438
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
  std::vector<Var> order = topo_order(root);
  for (Var& n : order)
    if (n.node->op) {
      std::lock_guard<std::mutex> lk(n.node->mu);
      n.node->grad.reset();
    }
  root.accumulate_grad(s);
  for (auto it = order.rbegin(); it != order.rend(); ++it) {
    Var& n = *it;
    if (!n.node->op) continue;
    std::optional<Tensor> up;
    {
      std::lock_guard<std::mutex> lk(n.node->mu);
      up = n.node->grad;
    }
    if (!up) err_invalid("internal: node reached in backward without a gradient");
    std::vector<bool> needs;
    for (const Var& in : n.node->inputs) needs.push_back(in.requires_grad());
    std::vector<std::optional<Tensor>> grads;
    if (retain_graph) {
      Vjp f;  // a copy: the node keeps its VJP for later passes
      {
        std::lock_guard<std::mutex> lk(n.node->mu);
        if (!n.node->vjp) err_invalid("internal: op node reached in backward without a VJP");
        f = *n.node->vjp;
      }
      grads = f(*up, needs);
    } else {
      Vjp f;
      {
        std::lock_guard<std::mutex> lk(n.node->mu);
        if (!n.node->vjp)
          err_invalid(
              "trying to backward through the graph a second time (or along an already freed path): pass "
              "retain_graph=True on the first backward call");
        f = std::move(*n.node->vjp);
        n.node->vjp.reset();
      }
      grads = f(*up, needs);
    }
    const std::vector<Var> inputs = n.node->inputs;
    for (size_t i = 0; i < inputs.size() && i < grads.size(); ++i) {
      if (!inputs[i].requires_grad() || !grads[i]) continue;
      inputs[i].accumulate_grad(unbroadcast(*grads[i], inputs[i].value().shape));
    }
  }
}

}  // namespace oxt
