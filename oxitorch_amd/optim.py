"""Optimizers and gradient clipping for oxitorch_amd.

Same surface as the reference module `oxitorch.optim`
(python/oxitorch/optim.py): `Sgd`, `AdamW`, `Adam` delegate to the host
core's `_native.RustSgd` / `_native.RustAdamW`, which keep every optimizer
buffer (velocities, moments, per-parameter step counters) on the device and
run each parameter's update as one HIP kernel over its flat slice
(`oxi_sgd_step` / `oxi_adamw_step`). A step rebinds the given Tensor objects
to their updated values, so the objects (and Parameter wrappers) keep their
identity across a run.

The reference's learning-rate schedules are host-side bookkeeping outside
the device hot path: their names exist and refuse to be made. Gradient
clipping computes its norms with the device reductions and rescales the
gradients on the device.
"""

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


# ---- learning-rate schedules ---------------------------------------------------

class _OutsideSchedule:
    """A learning-rate schedule of the reference (python/oxitorch/optim.py:104-226).
    Schedules only rewrite `optimizer.lr` between steps on the host, off the
    device hot path, so they are not part of this build: making one raises."""

    def __init__(self, *args, **kwargs):
        raise NotImplementedError(f"{type(self).__name__}: learning-rate schedules are outside this build's "
                                  "device hot path; set optimizer.lr between steps")


class StepLR(_OutsideSchedule):
    """Reference schedule (optim.py:133); refused."""


class CosineAnnealingLR(_OutsideSchedule):
    """Reference schedule (optim.py:145); refused."""


class LinearWarmup(_OutsideSchedule):
    """Reference schedule (optim.py:162); refused."""


class SequentialLR(_OutsideSchedule):
    """Reference schedule (optim.py:179); refused."""


class LambdaLR(_OutsideSchedule):
    """Reference schedule (optim.py:215); refused."""


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
