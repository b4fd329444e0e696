"""Optimizers, learning-rate schedules and gradient clipping for oxitorch_amd.

Same surface as the reference module `oxitorch.optim`
(python/oxitorch/optim.py): `Sgd`, `AdamW`, `Adam` delegate to the host
core's `_native.RustSgd` / `_native.RustAdamW`, which keep every optimizer
buffer (velocities, moments, per-parameter step counters) on the device and
run each parameter's update as one HIP kernel over its flat slice
(`oxi_sgd_step` / `oxi_adamw_step`). A step rebinds the given Tensor objects
to their updated values, so the objects (and Parameter wrappers) keep their
identity across a run.

Schedules only set `optimizer.lr`; the next device step reads it. Gradient
clipping computes its norms with the device reductions and rescales the
gradients on the device.
"""

import math

from oxitorch_amd import _native

__all__ = [
    "Adam",
    "AdamW",
    "CosineAnnealingLR",
    "LambdaLR",
    "LinearWarmup",
    "SequentialLR",
    "Sgd",
    "StepLR",
    "clip_grad_norm_",
    "clip_grad_value_",
]


def _tensor_of(p):
    """A Parameter wrapper's tensor, or the tensor itself."""
    return getattr(p, "tensor", p)


class _DeviceOptimizer:
    """torch-style `zero_grad()` / `step()` / mutable `lr` over a native
    optimizer (python/oxitorch/optim.py:18-49). The parameter list is read
    again at every call, so rebinding `opt.params` or a Parameter's tensor
    keeps the state of that list position."""

    def __init__(self, params, native):
        self.params = list(params)
        self._native = native

    @property
    def lr(self):
        return self._native.lr

    @lr.setter
    def lr(self, value):
        self._native.lr = value

    def _tensors(self):
        return [_tensor_of(p) for p in self.params]

    def zero_grad(self):
        self._native.zero_grad(self._tensors())

    def step(self):
        self._native.step(self._tensors())


class Sgd(_DeviceOptimizer):
    """SGD with optional (Nesterov) momentum (python/oxitorch/optim.py:52-65).

    buf = momentum*buf + g (buf starts at zero, so the first step uses g);
    p -= lr * (g + momentum*buf if nesterov else buf)."""

    def __init__(self, params, lr=0.01, momentum=0.0, nesterov=False):
        if nesterov and momentum <= 0.0:
            raise ValueError("nesterov momentum requires momentum > 0")
        self.momentum = momentum
        self.nesterov = nesterov
        super().__init__(params, _native.RustSgd(lr, momentum, nesterov))


class AdamW(_DeviceOptimizer):
    """Adam with decoupled weight decay (python/oxitorch/optim.py:68-83):
    p -= lr*weight_decay*p after the adaptive step. torch's defaults."""

    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2):
        self.betas = tuple(betas)
        self.eps = eps
        self.weight_decay = weight_decay
        super().__init__(params, _native.RustAdamW(lr, self.betas, eps, weight_decay, True))


class Adam(_DeviceOptimizer):
    """Classic Adam (python/oxitorch/optim.py:86-99): weight_decay*p is added
    to the gradient before the moments; no decay by default."""

    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0):
        self.betas = tuple(betas)
        self.eps = eps
        self.weight_decay = weight_decay
        super().__init__(params, _native.RustAdamW(lr, self.betas, eps, weight_decay, False))


# ---- learning-rate schedules (python/oxitorch/optim.py:104-243) ---------------

class _Schedule:
    """lr(epoch) = base_lr * factor(epoch). Building a schedule already applies
    epoch 0 (torch semantics); each `step()` moves to the next epoch."""

    def __init__(self, optimizer, last_epoch=-1):
        self.optimizer = optimizer
        self.base_lr = optimizer.lr
        self.last_epoch = last_epoch
        self.step()

    def _lr_factor(self, t):
        raise NotImplementedError

    def step(self):
        self.last_epoch += 1
        self.optimizer.lr = self.base_lr * self._lr_factor(self.last_epoch)

    def get_last_lr(self):
        return [self.optimizer.lr]


class StepLR(_Schedule):
    """Decay by `gamma` once every `step_size` epochs."""

    def __init__(self, optimizer, step_size, gamma=0.1, last_epoch=-1):
        self.step_size = step_size
        self.gamma = gamma
        super().__init__(optimizer, last_epoch)

    def _lr_factor(self, t):
        return self.gamma ** (t // self.step_size)


class CosineAnnealingLR(_Schedule):
    """Half-cosine from base_lr down to `eta_min` over `T_max` epochs."""

    def __init__(self, optimizer, T_max, eta_min=0.0, last_epoch=-1):
        self.T_max = T_max
        self.eta_min = eta_min
        super().__init__(optimizer, last_epoch)

    def _lr_factor(self, t):
        if self.T_max <= 0:
            return 1.0
        w = 0.5 * (1.0 + math.cos(math.pi * t / self.T_max))
        return (self.eta_min + (self.base_lr - self.eta_min) * w) / self.base_lr


class LinearWarmup(_Schedule):
    """Ramp linearly to base_lr over `warmup_epochs` ((t+1)/warmup), then hold."""

    def __init__(self, optimizer, warmup_epochs, last_epoch=-1):
        if warmup_epochs < 0:
            raise ValueError("warmup_epochs must be non-negative")
        self.warmup_epochs = warmup_epochs
        super().__init__(optimizer, last_epoch)

    def _lr_factor(self, t):
        return 1.0 if self.warmup_epochs == 0 else min(1.0, (t + 1) / self.warmup_epochs)


class LambdaLR(_Schedule):
    """lr = base_lr * lr_lambda(epoch)."""

    def __init__(self, optimizer, lr_lambda, last_epoch=-1):
        self.lr_lambda = lr_lambda
        super().__init__(optimizer, last_epoch)

    def _lr_factor(self, t):
        return self.lr_lambda(t)


class SequentialLR(_Schedule):
    """Hand over to the next schedule at each milestone epoch; a schedule
    counts its epochs from its own milestone. Every schedule is rebased on the
    first one's base_lr, whatever the order they were built in."""

    def __init__(self, optimizer, schedulers, milestones, last_epoch=-1):
        if len(schedulers) != len(milestones) + 1:
            raise ValueError(
                f"{len(schedulers)} schedulers need {len(schedulers) - 1} milestones, got {len(milestones)}"
            )
        self.schedulers = list(schedulers)
        self.milestones = list(milestones)
        base = self.schedulers[0].base_lr
        for s in self.schedulers:
            s.base_lr = base
        self.optimizer = optimizer
        self.base_lr = base
        self.last_epoch = last_epoch
        self.step()

    def step(self):
        self.last_epoch += 1
        t = self.last_epoch
        k = sum(1 for m in self.milestones if t >= m)
        start = self.milestones[k - 1] if k else 0
        self.optimizer.lr = self.base_lr * self.schedulers[k]._lr_factor(t - start)


# ---- gradient clipping (python/oxitorch/optim.py:248-299) ----------------------

def _with_grads(params):
    for p in params:
        t = _tensor_of(p)
        g = t.grad
        if g is not None:
            yield t, g


def clip_grad_norm_(params, max_norm, norm_type=2.0):
    """Scale all gradients by max_norm/(total+1e-6) when their joint p-norm
    `total` exceeds max_norm; returns the pre-clip total as a float. Norms
    and scaling run on the device; `norm_type` is any p >= 1 or inf."""
    pairs = list(_with_grads(list(params)))
    if norm_type == float("inf"):
        total = max((float(g.apply("abs").max().item()) for _, g in pairs), default=0.0)
    else:
        acc = 0.0
        for _, g in pairs:
            acc += float((g.apply("abs") ** float(norm_type)).sum().item())
        total = acc ** (1.0 / norm_type)
    scale = max_norm / (total + 1e-6)
    if scale < 1.0:
        for t, g in pairs:
            t.grad = g * scale
    return total


def clip_grad_value_(params, clip_value):
    """Clamp every gradient element to [-clip_value, clip_value] on the device."""
    clip_value = float(clip_value)
    if clip_value <= 0:
        raise ValueError("clip_value must be positive")
    for t, g in _with_grads(list(params)):
        t.grad = _native.clamp(g, -clip_value, clip_value)
