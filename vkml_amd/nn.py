"""Layers for the BASELINE training configs, mirroring vkML's python/vkml/nn.py:
Module, Linear, Conv2d, MaxPool2d, Flatten, ReLU, Sequential, and the
cross-entropy loss. Weights use torch's Kaiming-uniform default, bound
1/sqrt(fan_in), drawn from a seedable numpy generator exactly as the reference
draws them (nn.py:31-44, 253-301, 659-700): weight first, then bias.
"""
from __future__ import annotations

import math

import numpy as np

from . import tensor as T

_INIT_RNG = np.random.default_rng()


def manual_seed(seed: int) -> None:
    """Make subsequent weight initialisation reproducible (reference nn.py:34-44)."""
    global _INIT_RNG
    _INIT_RNG = np.random.default_rng(seed)


def _pair(v):
    return (int(v[0]), int(v[1])) if isinstance(v, (tuple, list)) else (int(v), int(v))


class Module:
    backend = None

    def __init__(self):
        object.__setattr__(self, "_parameters", {})
        object.__setattr__(self, "_modules", {})

    def __setattr__(self, name, value):
        if isinstance(value, T.Tensor) and value.requires_grad:
            self._parameters[name] = value
        elif isinstance(value, Module):
            self._modules[name] = value
        object.__setattr__(self, name, value)

    def parameters(self) -> list[T.Tensor]:
        out = list(self._parameters.values())
        for m in self._modules.values():
            out.extend(m.parameters())
        return out

    def __call__(self, *args):
        return self.forward(*args)

    def forward(self, *args):
        raise NotImplementedError


class Linear(Module):
    """y = x @ W^T + b with W stored (out, in) (reference nn.py:253-301)."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True, backend=None):
        super().__init__()
        bound = 1.0 / math.sqrt(in_features)
        w = _INIT_RNG.uniform(-bound, bound, size=(out_features, in_features)).astype(np.float32)
        self.weight = T.tensor(w, requires_grad=True, backend=backend)
        self.bias = None
        if bias:
            b = _INIT_RNG.uniform(-bound, bound, size=(out_features,)).astype(np.float32)
            self.bias = T.tensor(b, requires_grad=True, backend=backend)

    def forward(self, x: T.Tensor) -> T.Tensor:
        y = T.matmul(x, self.weight.transpose(-2, -1))
        return y + self.bias if self.bias is not None else y


class Conv2d(Module):
    """im2col convolution, weight (out, in, kh, kw) (reference nn.py:659-700)."""

    def __init__(self, in_channels: int, out_channels: int, kernel_size, stride=1, padding=0,
                 dilation=1, bias: bool = True, backend=None):
        super().__init__()
        self.kernel_size = _pair(kernel_size)
        self.stride, self.padding, self.dilation = _pair(stride), _pair(padding), _pair(dilation)
        fan_in = in_channels * self.kernel_size[0] * self.kernel_size[1]
        bound = 1.0 / math.sqrt(fan_in)
        w = _INIT_RNG.uniform(-bound, bound,
                              size=(out_channels, in_channels, *self.kernel_size)).astype(np.float32)
        self.weight = T.tensor(w, requires_grad=True, backend=backend)
        self.bias = None
        if bias:
            b = _INIT_RNG.uniform(-bound, bound, size=(out_channels,)).astype(np.float32)
            self.bias = T.tensor(b, requires_grad=True, backend=backend)

    def forward(self, x: T.Tensor) -> T.Tensor:
        return T.conv2d(x, self.weight, self.bias, self.stride, self.padding, self.dilation)


class MaxPool2d(Module):
    def __init__(self, kernel_size, stride=None, padding=0):
        super().__init__()
        self.kernel_size = _pair(kernel_size)
        self.stride = self.kernel_size if stride is None else _pair(stride)
        self.padding = _pair(padding)

    def forward(self, x):
        return T.max_pool2d(x, self.kernel_size, self.stride, self.padding)


class Flatten(Module):
    """contiguous() then reshape (reference nn.py:581-600)."""

    def __init__(self, start_dim: int = 1):
        super().__init__()
        self.start_dim = start_dim

    def forward(self, x):
        head = list(x.shape[: self.start_dim])
        tail = 1
        for d in x.shape[self.start_dim:]:
            tail *= d
        return x.contiguous().reshape(head + [tail])


class ReLU(Module):
    def forward(self, x):
        return T.relu(x)


class Sequential(Module):
    def __init__(self, *layers):
        super().__init__()
        for i, layer in enumerate(layers):
            setattr(self, f"l{i}", layer)
        object.__setattr__(self, "layers", list(layers))

    def forward(self, x):
        for layer in self.layers:
            x = layer(x)
        return x


def cross_entropy(logits: T.Tensor, target: T.Tensor) -> T.Tensor:
    return T.cross_entropy(logits, target)
