"""Modules of the drop-in surface (the interface of
python/oxitorch/nn/module.py:11-122).

A module's state is found by one walk over its attributes in insertion
order: a Parameter attribute is a leaf, a Module attribute is entered, and a
list or tuple attribute contributes its Parameter and Module items under
their index. The walk names every entry with its dotted path
(`layers.0.weight`); those paths are the keys of `state_dict()` and
`load_state_dict()`, so checkpoints keep the reference's key format.
"""

import numpy as np


class Parameter:
    """A trainable tensor: what the module walk collects."""

    __slots__ = ("tensor",)

    def __init__(self, tensor):
        self.tensor = tensor

    @property
    def grad(self):
        return self.tensor.grad

    def zero_grad(self):
        self.tensor.zero_grad()

    def detach_numpy(self):
        return self.tensor.detach().numpy()


def _entries(owner, prefix):
    """(path, Parameter | Module) for the state held directly by `owner`."""
    for name, value in vars(owner).items():
        if isinstance(value, (Parameter, Module)):
            yield prefix + name, value
        elif isinstance(value, (list, tuple)):
            for i, item in enumerate(value):
                if isinstance(item, (Parameter, Module)):
                    yield f"{prefix}{name}.{i}", item


class Module:
    training = True

    def _walk(self, prefix=""):
        """Every parameter and submodule below this one, depth first."""
        for path, value in _entries(self, prefix):
            yield path, value
            if isinstance(value, Module):
                yield from value._walk(path + ".")

    def named_parameters(self, prefix=""):
        return ((path, p) for path, p in self._walk(prefix) if isinstance(p, Parameter))

    def parameters(self):
        return [p for _, p in self.named_parameters()]

    def modules(self):
        """This module and every submodule below it."""
        return [self] + [m for _, m in self._walk() if isinstance(m, Module)]

    def zero_grad(self):
        for p in self.parameters():
            p.zero_grad()

    def train(self, mode=True):
        """Sets the training flag here and on every submodule, lists included."""
        for m in self.modules():
            m.training = mode
        return self

    def eval(self):
        return self.train(False)

    def state_dict(self):
        return {path: p.detach_numpy() for path, p in self.named_parameters()}

    def load_state_dict(self, state):
        """Replaces every parameter with the value under its path in `state`
        (a state_dict() mapping), as a new leaf that requires grad, uploaded
        through the staging ring. Every key and shape is checked before any
        parameter changes: a missing key raises KeyError, a shape that
        differs raises ValueError."""
        from . import functional

        staged = []
        for path, p in self.named_parameters():
            if path not in state:
                raise KeyError(f"missing key in state_dict: {path!r}")
            value = np.asarray(state[path])
            want = list(p.tensor.shape)
            if list(value.shape) != want:
                raise ValueError(f"shape mismatch for {path!r}: state {list(value.shape)} vs parameter {want}")
            staged.append((p, value))
        for p, value in staged:
            p.tensor = functional._native_from_numpy(value, requires_grad=True)

    def forward(self, *args, **kwargs):
        raise NotImplementedError(f"{type(self).__name__} defines no forward")

    def __call__(self, *args, **kwargs):
        return self.forward(*args, **kwargs)


class Sequential(Module):
    """Applies its layers in order."""

    def __init__(self, *layers):
        self.layers = list(layers)

    def forward(self, x):
        for layer in self.layers:
            x = layer(x)
        return x

    def __getitem__(self, index):
        return self.layers[index]
