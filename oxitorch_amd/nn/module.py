"""Module base classes (the interface of python/oxitorch/nn/module.py:11-122):
a Parameter marks a trainable tensor; a Module collects the Parameters of its
attributes and submodules in insertion order."""


class Parameter:
    """A named, trainable tensor (`tensor.requires_grad` is True)."""

    def __init__(self, tensor):
        self.tensor = tensor

    @property
    def grad(self):
        return self.tensor.grad

    def zero_grad(self):
        self.tensor.zero_grad()

    def detach_numpy(self):
        return self.tensor.detach().numpy()


class Module:
    training = True

    def parameters(self):
        return [p for _, p in self.named_parameters()]

    def named_parameters(self, prefix=""):
        for name, v in self.__dict__.items():
            if isinstance(v, Parameter):
                yield prefix + name, v
            elif isinstance(v, Module):
                yield from v.named_parameters(prefix + name + ".")
            elif isinstance(v, (list, tuple)):
                for i, item in enumerate(v):
                    if isinstance(item, Module):
                        yield from item.named_parameters(f"{prefix}{name}.{i}.")
                    elif isinstance(item, Parameter):
                        yield f"{prefix}{name}.{i}", item

    def zero_grad(self):
        for p in self.parameters():
            p.zero_grad()

    def train(self, mode=True):
        self.training = mode
        for v in self.__dict__.values():
            if isinstance(v, Module):
                v.train(mode)
        return self

    def eval(self):
        return self.train(False)

    def state_dict(self):
        return {name: p.detach_numpy() for name, p in self.named_parameters()}

    def forward(self, *args, **kwargs):
        raise NotImplementedError

    def __call__(self, *args, **kwargs):
        return self.forward(*args, **kwargs)


class Sequential(Module):
    def __init__(self, *layers):
        self.layers = list(layers)

    def forward(self, x):
        for layer in self.layers:
            x = layer(x)
        return x
