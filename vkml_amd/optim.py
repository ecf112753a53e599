"""SGD with momentum, weight decay and Nesterov, mirroring vkML's
python/vkml/optim.py:79-199.

The reference builds one step as three batched passes of ScaledAdd nodes
(realise every new velocity, then every new parameter value, then assign them
back in place): with gradient g' = g + p*wd (weight decay), velocity
v = m*v + g' (v = g' on the first step), direction v or, for Nesterov,
g' + m*v, and p = p - lr*direction, each `a*alpha + b*beta` being two rounded
products and one rounded add.

`SGD(..., fused=True)` (the default) computes exactly those values with one
backend call for all parameters (`vkhip_sgd_step`: one launch, in place),
instead of two nodes per parameter; `fused=False` builds the reference's node
graph. Both give bit-identical parameters.
"""
from __future__ import annotations

import numpy as np

from . import tensor as T


class SGD:
    def __init__(self, params, lr: float = 1e-2, momentum: float = 0.0,
                 weight_decay: float = 0.0, nesterov: bool = False, fused: bool = True):
        self.params = list(params)
        if not self.params:
            raise ValueError("optimizer received an empty parameter list")
        for p in self.params:
            if not p.requires_grad:
                raise ValueError("optimizer received a parameter with requires_grad=False")
        if nesterov and momentum == 0.0:
            raise ValueError("nesterov momentum requires momentum != 0")
        self.lr = lr
        self.momentum = momentum
        self.weight_decay = weight_decay
        self.nesterov = nesterov
        self.fused = fused
        self._velocity = [None] * len(self.params)  # Tensors (node path)
        self._vbuf = [None] * len(self.params)      # (buffer, byte offset), fused path

    def zero_grad(self) -> None:
        for p in self.params:
            p.grad = None

    def step(self) -> None:
        with T.no_grad():
            live = [(i, p, p.grad) for i, p in enumerate(self.params) if p.grad is not None]
            if not live:
                return
            backend = live[0][1].node.backend
            if (self.fused and hasattr(backend, "sgd_step")
                    and all(self._fusable(p, g, backend) for _, p, g in live)):
                self._fused_step(live, backend)
            else:
                self._node_step(live)

    # -- the reference's graph: two ScaledAdd nodes and an assign per parameter --
    def _gradient(self, p, g):
        # The reference's grad + param * decay (optim.py:134-142), as one
        # ScaledAdd node: g*1 + p*decay is the same two roundings.
        if self.weight_decay == 0.0:
            return g
        return T.scaled_add(g, p.detach(), 1.0, self.weight_decay)

    def _node_step(self, live) -> None:
        plans = []
        for i, p, g in live:
            g = self._gradient(p, g)
            if self.momentum == 0.0:
                plans.append((i, p, None, g))
                continue
            prev = self._velocity[i]
            if prev is None and self._vbuf[i] is not None:  # state left by a fused step
                node = T.Node(T.INPUT, p.shape, np.float32, p.node.backend)
                node.storage, node.offset, node.computed = self._vbuf[i][0], self._vbuf[i][1] // 4, True
                prev = T.Tensor(node)
                self._vbuf[i] = None
            v = g if prev is None else T.scaled_add(prev, g, self.momentum, 1.0)
            plans.append((i, p, v, g))
        T.realize([v for _, _, v, _ in plans if v is not None])
        values = []
        for i, p, v, g in plans:
            if v is None:
                direction = g
            else:
                self._velocity[i] = v.detach()
                direction = (T.scaled_add(g, self._velocity[i], 1.0, self.momentum)
                             if self.nesterov else self._velocity[i])
            values.append(T.scaled_add(p.detach(), direction, 1.0, -self.lr))
        T.realize(values)
        T.assign([p for _, p, _, _ in plans], values)

    # -- one backend call --------------------------------------------------------
    @staticmethod
    def _fusable(p, g, backend) -> bool:
        return (p.dtype == np.float32 and g.dtype == np.float32 and p.shape == g.shape
                and g.node.backend is backend and p.node.computed and p.node.is_contiguous()
                and p.node.offset == 0)

    def _fused_step(self, live, backend) -> None:
        grads = [g.contiguous() for _, _, g in live]
        T.realize(grads)
        entries = []
        for (i, p, _), g in zip(live, grads):
            n = T._numel(p.shape)
            first = False
            vbuf = None
            if self.momentum != 0.0:
                if self._vbuf[i] is None:
                    if self._velocity[i] is not None:  # state left by the node path
                        vt = self._velocity[i].contiguous()
                        T.realize([vt])
                        self._vbuf[i] = (vt.node.storage, vt.node.offset * 4)
                    else:
                        self._vbuf[i] = (backend.alloc(max(n, 1) * 4), 0)
                        first = True
                vbuf = self._vbuf[i]
            entries.append((p.node.storage, g.node.storage, g.node.offset * 4,
                            vbuf[0] if vbuf else None, vbuf[1] if vbuf else 0, n, first))
        backend.sgd_step(entries, self.lr, self.momentum, self.weight_decay, self.nesterov)
        self._velocity = [None] * len(self.params)
