// Optimizers of the host core: Sgd and AdamW over device parameters
// (crates/oxi-autograd/src/optim.rs). The element math runs in the
// oxi_sgd_step / oxi_adamw_step kernels; this file owns the per-index state,
// the step counters and the parameter rebinding.
#include <string>

#include "host.h"

namespace oxt {
namespace {

// slot (optim.rs:31-51): grow the slot list to cover `index`, create a zero
// buffer of `len` floats on first use, reject a parameter whose size changed.
Tensor& slot(std::vector<std::optional<Tensor>>& slots, size_t index, int64_t len) {
  if (slots.size() <= index) slots.resize(index + 1);
  if (!slots[index]) slots[index] = t_zeros({len}, Dev::Hip);
  const int64_t have = slots[index]->numel();
  if (have != len)
    err_invalid("optimizer state for parameter " + std::to_string(index) + " has " + std::to_string(have) +
                " elements but the parameter now has " + std::to_string(len) +
                "; the parameter set changed mid-run");
  return *slots[index];
}

// bump_step (optim.rs:54-60).
uint64_t bump_step(std::vector<uint64_t>& steps, size_t index) {
  if (steps.size() <= index) steps.resize(index + 1, 0);
  return ++steps[index];
}

struct Operands {
  Tensor value, grad;
};

// Row-major value and gradient of a parameter on the device (the reference
// reads both with to_vec, optim.rs:108,129).
Operands operands(const Var& param, const Tensor& grad, const char* what) {
  const Tensor& val = param.value();
  require_hip(val, what);
  require_hip(grad, what);
  if (grad.numel() != val.numel()) err_shape(fmt_shape(grad.shape), fmt_shape(val.shape));
  return {t_contiguous(val), t_contiguous(grad)};
}

}  // namespace

// Sgd::step_param (optim.rs:104-137).
void Sgd::step_param(size_t index, Var& param) {
  const std::optional<Tensor> grad = param.grad();
  if (!grad) return;
  const Operands op = operands(param, *grad, "SGD step");
  const int64_t n = op.value.numel();
  float* buf = nullptr;
  if (momentum_ > 0.0f) buf = slot(velocities_, index, n).data();
  Tensor out = Tensor::empty(op.value.shape, Dev::Hip);
  hip_check(oxi_sgd_step(op.value.data(), op.grad.data(), buf, out.data(), n, lr_, momentum_,
                         nesterov_ && momentum_ > 0.0f ? 1 : 0));
  param = Var::leaf(std::move(out), true);  // rewrap_leaf (optim.rs:24-28)
}

// Sgd::step (optim.rs:143-148): every parameter with a gradient in one
// multi-slice call. Parameters are prepared in list order; an error at one
// leaves the earlier ones stepped, as the reference's loop does.
void Sgd::step(std::vector<Var*>& params) {
  std::vector<oxi_sgd_slice> slices;
  std::vector<std::pair<Var*, Tensor>> outs;
  std::vector<Operands> keep;  // operands stay alive until the launch is queued
  auto flush = [&]() {
    if (slices.empty()) return;
    hip_check(oxi_sgd_step_multi(slices.data(), (int)slices.size(), lr_, momentum_,
                                 nesterov_ && momentum_ > 0.0f ? 1 : 0));
    for (auto& [var, out] : outs) *var = Var::leaf(std::move(out), true);
    slices.clear();
    outs.clear();
  };
  for (size_t i = 0; i < params.size(); ++i) {
    const std::optional<Tensor> grad = params[i]->grad();
    if (!grad) continue;
    try {
      keep.push_back(operands(*params[i], *grad, "SGD step"));
      const Operands& op = keep.back();
      const int64_t n = op.value.numel();
      float* buf = momentum_ > 0.0f ? slot(velocities_, i, n).data() : nullptr;
      Tensor out = Tensor::empty(op.value.shape, Dev::Hip);
      slices.push_back({op.value.data(), op.grad.data(), buf, out.data(), n});
      outs.emplace_back(params[i], std::move(out));
    } catch (...) {
      flush();
      throw;
    }
  }
  flush();
}

// AdamW::step_param (optim.rs:223-262).
void AdamW::step_param(size_t index, Var& param) {
  const std::optional<Tensor> grad = param.grad();
  if (!grad) return;
  const Operands op = operands(param, *grad, "AdamW step");
  const int64_t n = op.value.numel();
  // the counter advances before the state-size check, as in the reference
  const uint64_t t = bump_step(steps_, index);
  Tensor& m = slot(moments_, index, n);
  Tensor& v = slot(sq_moments_, index, n);
  Tensor out = Tensor::empty(op.value.shape, Dev::Hip);
  hip_check(oxi_adamw_step(op.value.data(), op.grad.data(), m.data(), v.data(), out.data(), n, lr_, beta1_, beta2_,
                           eps_, wd_, decoupled_ ? 1 : 0, (int64_t)t));
  param = Var::leaf(std::move(out), true);
}

// AdamW::step (optim.rs:267-272), batched like Sgd::step.
void AdamW::step(std::vector<Var*>& params) {
  std::vector<oxi_adamw_slice> slices;
  std::vector<std::pair<Var*, Tensor>> outs;
  std::vector<Operands> keep;
  auto flush = [&]() {
    if (slices.empty()) return;
    hip_check(oxi_adamw_step_multi(slices.data(), (int)slices.size(), lr_, beta1_, beta2_, eps_, wd_,
                                   decoupled_ ? 1 : 0));
    for (auto& [var, out] : outs) *var = Var::leaf(std::move(out), true);
    slices.clear();
    outs.clear();
  };
  for (size_t i = 0; i < params.size(); ++i) {
    const std::optional<Tensor> grad = params[i]->grad();
    if (!grad) continue;
    try {
      keep.push_back(operands(*params[i], *grad, "AdamW step"));
      const Operands& op = keep.back();
      const int64_t n = op.value.numel();
      const uint64_t t = bump_step(steps_, i);
      Tensor& m = slot(moments_, i, n);
      Tensor& v = slot(sq_moments_, i, n);
      Tensor out = Tensor::empty(op.value.shape, Dev::Hip);
      slices.push_back({op.value.data(), op.grad.data(), m.data(), v.data(), out.data(), n, (int64_t)t});
      outs.emplace_back(params[i], std::move(out));
    } catch (...) {
      flush();
      throw;
    }
  }
  flush();
}

}  // namespace oxt
