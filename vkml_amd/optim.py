"""SGD with momentum, mirroring vkML's python/vkml/optim.py:79-199.

One step is three batched passes, as in the reference: realise every new
velocity, then every new parameter value, then assign the values back. Each
update is a single ScaledAdd node: v = m*v + g, p = 1*p + (-lr)*v (the first
step's velocity is the gradient itself).
"""
from __future__ import annotations

from . import tensor as T


class SGD:
    def __init__(self, params, lr: float = 1e-2, momentum: float = 0.0):
        self.params = list(params)
        self.lr = lr
        self.momentum = momentum
        self._velocity = [None] * len(self.params)

    def zero_grad(self) -> None:
        for p in self.params:
            p.grad = None

    def step(self) -> None:
        with T.no_grad():
            plans = []
            for i, p in enumerate(self.params):
                g = p.grad
                if g is None:
                    continue
                if self.momentum == 0.0:
                    plans.append((i, p, None, g))
                    continue
                prev = self._velocity[i]
                v = g if prev is None else T.scaled_add(prev, g, self.momentum, 1.0)
                plans.append((i, p, v, g))
            state = [v for _, _, v, _ in plans if v is not None]
            T.realize(state)
            values = []
            for i, p, v, g in plans:
                if v is not None:
                    self._velocity[i] = v.detach()
                    direction = self._velocity[i]
                else:
                    direction = g
                values.append(T.scaled_add(p.detach(), direction, 1.0, -self.lr))
            T.realize(values)
            T.assign([p for _, p, _, _ in plans], values)
