"""Shared test configuration.

Markers:
  gpu -- needs an MI355X (gfx950) and the built libvkhip.so; the parity tests.
Everything unmarked runs on a CPU-only machine: the oracle against the
reference's golden vectors and closed forms, host-side planning logic, and the
C-ABI library's symbol table (no device calls).
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

# The reference suite's session seed (tests/python/test_vulkan_kernels.py:32).
SEED = 20260726
FP32_EPS = float(np.finfo(np.float32).eps)
PAIRWISE_BLOCK = 32


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")


def pairwise_gamma(n: int) -> float:
    """Relative error factor of pairwise summation of n terms (reference
    tests/python/tolerance.py:310-318): (B + log2(n/B)) * eps."""
    if n <= 1:
        return 0.0
    return (PAIRWISE_BLOCK + np.log2(max(n / PAIRWISE_BLOCK, 1.0))) * FP32_EPS


def gemm_atol(a: np.ndarray, b: np.ndarray, safety: float = 16.0) -> float:
    """Backward-error bound for a product (reference conftest.py:145-165):
    gamma(K) * max_ij sum_k |a_ik b_kj| * safety."""
    k = a.shape[-1]
    abs_prod = np.abs(a.astype(np.float64)) @ np.abs(b.astype(np.float64))
    return float(pairwise_gamma(max(k, 32)) * abs_prod.max() * safety)


def normwise_rel_err(got: np.ndarray, want: np.ndarray) -> float:
    """max |got - want| / max |want|: the north-star's relative error, normwise
    (elementwise relative error is meaningless near the zeros of C)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    scale = float(np.max(np.abs(want))) if want.size else 0.0
    if scale == 0.0:
        return float(np.max(np.abs(got))) if got.size else 0.0
    return float(np.max(np.abs(got - want)) / scale)


def gemm_tolerance(k: int) -> float:
    """North-star GEMM/softmax gate: max relative error 1e-5 * sqrt(K)."""
    return 1e-5 * float(np.sqrt(max(k, 1)))


@pytest.fixture(scope="session")
def rng():
    return np.random.default_rng(SEED)


@pytest.fixture(scope="session")
def hip():
    """The process-wide HIP backend; GPU tests only."""
    from vkml_amd.device import backend

    return backend()


# ---- cross-entropy helpers shared by the host-core and device training tests ----

def ce_loss_and_grad(backend, logits, labels, fused):
    """cross_entropy's loss and logits gradient on `backend`, built as the
    fused CROSS_ENTROPY nodes (fused=True) or as the reference composition."""
    from vkml_amd import tensor as T

    prev = T.FUSED_CROSS_ENTROPY
    T.FUSED_CROSS_ENTROPY = fused
    try:
        x = T.tensor(logits, requires_grad=True, backend=backend)
        loss = T.cross_entropy(x, T.tensor(labels, backend=backend))
        loss.backward()
        return loss.numpy(), x.grad.numpy()
    finally:
        T.FUSED_CROSS_ENTROPY = prev


def conv_loss_and_grads(backend, x, w, bias, stride, pad, dil, implicit, x_grad=True, fold=None,
                        fused_dx=None):
    """sum(conv2d(x, w, bias) * probe) and the gradients of x, w and bias on
    `backend`, with conv2d built as one CONV2D node (implicit=True) or as the
    reference's im2col + matmul graph. `probe` is a fixed pattern so every
    output position carries a different weight into the gradients. `fold`
    overrides FOLD_CONV_WEIGHT_GRAD (the weight gradient as one batch-summed
    node, or per-image node + batch SUM) and `fused_dx` FUSED_CONV_INPUT_GRAD
    (the input gradient as one node, or TN product + COL2IM) when not None."""
    from vkml_amd import tensor as T

    prev = T.IMPLICIT_CONV
    prev_fold = T.FOLD_CONV_WEIGHT_GRAD
    prev_dx = T.FUSED_CONV_INPUT_GRAD
    T.IMPLICIT_CONV = implicit
    if fold is not None:
        T.FOLD_CONV_WEIGHT_GRAD = fold
    if fused_dx is not None:
        T.FUSED_CONV_INPUT_GRAD = fused_dx
    try:
        xt = T.tensor(x, requires_grad=x_grad, backend=backend)
        wt = T.tensor(w, requires_grad=True, backend=backend)
        bt = T.tensor(bias, requires_grad=True, backend=backend)
        out = T.conv2d(xt, wt, bt, stride, pad, dil)
        probe = np.linspace(-1.0, 1.0, int(np.prod(out.shape)), dtype=np.float32)
        loss = T.sum(out * T.tensor(probe.reshape(out.shape), backend=backend))
        loss.backward()
        return (out.numpy(), xt.grad.numpy() if x_grad else None, wt.grad.numpy(),
                bt.grad.numpy())
    finally:
        T.IMPLICIT_CONV = prev
        T.FOLD_CONV_WEIGHT_GRAD = prev_fold
        T.FUSED_CONV_INPUT_GRAD = prev_dx


def conv_relu_loss_and_grads(backend, x, w, bias, stride, pad, dil, fused):
    """sum(relu(conv2d(x, w, bias)) * probe) and the gradients of x, w and bias,
    with relu(conv + bias) built as one CONV2D_BIAS_RELU node (fused) or as
    the CONV2D, ADD and RELU nodes."""
    from vkml_amd import tensor as T

    prev = T.FUSED_CONV_EPILOGUE
    T.FUSED_CONV_EPILOGUE = fused
    try:
        xt = T.tensor(x, requires_grad=True, backend=backend)
        wt = T.tensor(w, requires_grad=True, backend=backend)
        bt = T.tensor(bias, requires_grad=True, backend=backend)
        out = T.relu(T.conv2d(xt, wt, bt, stride, pad, dil))
        assert (out.node.op == T.OP["CONV2D_BIAS_RELU"]) == fused
        probe = np.linspace(-1.0, 1.0, int(np.prod(out.shape)), dtype=np.float32)
        loss = T.sum(out * T.tensor(probe.reshape(out.shape), backend=backend))
        loss.backward()
        return out.numpy(), xt.grad.numpy(), wt.grad.numpy(), bt.grad.numpy()
    finally:
        T.FUSED_CONV_EPILOGUE = prev


def relu_pool_loss_and_grad(backend, x, kernel, stride, pad, fused):
    """sum(max_pool2d(relu(x)) * probe) and the gradient of x, with the relu
    and pool gradients built as one MAX_POOL2D_BACKWARD_RELU node (fused) or
    as MAX_POOL2D_BACKWARD and RELU_BACKWARD."""
    from vkml_amd import tensor as T

    prev = T.FUSED_POOL_RELU_GRAD
    T.FUSED_POOL_RELU_GRAD = fused
    try:
        xt = T.tensor(x, requires_grad=True, backend=backend)
        out = T.max_pool2d(T.relu(xt), kernel, stride, pad)
        probe = np.linspace(-1.0, 1.0, int(np.prod(out.shape)), dtype=np.float32)
        loss = T.sum(out * T.tensor(probe.reshape(out.shape), backend=backend))
        loss.backward()
        want = T.OP["MAX_POOL2D_BACKWARD_RELU"] if fused else T.OP["RELU_BACKWARD"]
        assert xt.grad.node.op == want
        return out.numpy(), xt.grad.numpy()
    finally:
        T.FUSED_POOL_RELU_GRAD = prev


def conv_pool_loss_and_grads(backend, x, w, bias, fused):
    """sum(max_pool2d(relu(conv2d(x, w, bias, pad 1)), 2) * probe) with x
    needing no gradient, and the weight and bias gradients: built as one
    CONV2D_POOL_WEIGHT_BIAS_GRAD node (fused) or as MAX_POOL2D_BACKWARD_RELU,
    CONV2D_WEIGHT_GRAD_SUM and the bias's SUM."""
    from vkml_amd import tensor as T

    prev = T.FUSED_CONV_POOL_GRAD
    T.FUSED_CONV_POOL_GRAD = fused
    try:
        xt = T.tensor(x, backend=backend)
        wt = T.tensor(w, requires_grad=True, backend=backend)
        bt = T.tensor(bias, requires_grad=True, backend=backend)
        out = T.max_pool2d(T.relu(T.conv2d(xt, wt, bt, 1, 1, 1)), 2)
        probe = np.linspace(-1.0, 1.0, int(np.prod(out.shape)), dtype=np.float32)
        loss = T.sum(out * T.tensor(probe.reshape(out.shape), backend=backend))
        loss.backward()
        src = wt.grad.node
        while src.view_src is not None:
            src = src.view_src
        assert (src.op == T.OP["CONV2D_POOL_WEIGHT_BIAS_GRAD"]) == fused
        return out.numpy(), wt.grad.numpy(), bt.grad.numpy()
    finally:
        T.FUSED_CONV_POOL_GRAD = prev


def pool_bias_loss_and_grads(backend, x, w, bias, fused):
    """sum(max_pool2d(relu(conv2d(x, w, bias, pad 1)), 2) * probe) with x
    needing its gradient: the x, weight and bias gradients, the bias's built as
    one MAX_POOL2D_BACKWARD_RELU_BIAS node with the pool gradient (fused) or as
    MAX_POOL2D_BACKWARD_RELU and SUM."""
    from vkml_amd import tensor as T

    prev = T.FUSED_POOL_BIAS_GRAD
    T.FUSED_POOL_BIAS_GRAD = fused
    try:
        xt = T.tensor(x, requires_grad=True, backend=backend)
        wt = T.tensor(w, requires_grad=True, backend=backend)
        bt = T.tensor(bias, requires_grad=True, backend=backend)
        out = T.max_pool2d(T.relu(T.conv2d(xt, wt, bt, 1, 1, 1)), 2)
        probe = np.linspace(-1.0, 1.0, int(np.prod(out.shape)), dtype=np.float32)
        loss = T.sum(out * T.tensor(probe.reshape(out.shape), backend=backend))
        loss.backward()
        src = bt.grad.node
        while src.view_src is not None:
            src = src.view_src
        assert (src.op == T.OP["MAX_POOL2D_BACKWARD_RELU_BIAS"]) == fused
        return out.numpy(), xt.grad.numpy(), wt.grad.numpy(), bt.grad.numpy()
    finally:
        T.FUSED_POOL_BIAS_GRAD = prev


def conv_pool_node(backend, x, y, gp, kernel, pad):
    """The CONV2D_POOL_WEIGHT_BIAS_GRAD node alone over given x, y and gp
    (unit stride and dilation): its [Cout*C*kh*kw + Cout] output."""
    from vkml_amd import tensor as T

    n_, c, h, w_ = x.shape
    cout = y.shape[1]
    ck = c * kernel[0] * kernel[1]
    xt, yt, gt = (T.tensor(a, backend=backend) for a in (x, y, gp))
    node = T.Node(T.OP["CONV2D_POOL_WEIGHT_BIAS_GRAD"], (cout * ck + cout,), np.float32, xt.node.backend,
                  [xt.node, yt.node, gt.node], params=T._unfold_params(kernel, (1, 1), pad, (1, 1), (h, w_)))
    return T.Tensor(node).numpy()


def linear_loss_and_grads(backend, x, w, bias, relu, fused):
    """sum(relu?(x @ w.T + bias) * probe) and the gradients of x, w and bias,
    with the product, bias add and relu built as one MATMUL_BIAS node (fused)
    or as the MATMUL, ADD and RELU nodes."""
    from vkml_amd import tensor as T

    prev = T.FUSED_LINEAR_BIAS
    T.FUSED_LINEAR_BIAS = fused
    try:
        xt = T.tensor(x, requires_grad=True, backend=backend)
        wt = T.tensor(w, requires_grad=True, backend=backend)
        bt = T.tensor(bias, requires_grad=True, backend=backend)
        out = T.matmul(xt, wt.transpose(-2, -1)) + bt
        if relu:
            out = T.relu(out)
        assert (out.node.view_src is not None and out.node.view_src.op == T.OP["MATMUL_BIAS"]) == fused
        probe = np.linspace(-1.0, 1.0, int(np.prod(out.shape)), dtype=np.float32)
        loss = T.sum(out * T.tensor(probe.reshape(out.shape), backend=backend))
        loss.backward()
        return out.numpy(), xt.grad.numpy(), wt.grad.numpy(), bt.grad.numpy()
    finally:
        T.FUSED_LINEAR_BIAS = prev


def mlp2_loss_and_grads(backend, x, w1, b1, w2, fused):
    """sum((relu(x @ w1.T + b1) @ w2.T) * probe) and the gradients of x, w1,
    b1 and w2, with the hidden relu's gradient built as one
    MATMUL_RELU_BACKWARD node over the second layer's input-gradient product
    (fused) or as MATMUL then RELU_BACKWARD."""
    from vkml_amd import tensor as T

    prev = T.FUSED_MATMUL_RELU_GRAD
    T.FUSED_MATMUL_RELU_GRAD = fused
    try:
        xt = T.tensor(x, requires_grad=True, backend=backend)
        w1t = T.tensor(w1, requires_grad=True, backend=backend)
        b1t = T.tensor(b1, requires_grad=True, backend=backend)
        w2t = T.tensor(w2, requires_grad=True, backend=backend)
        h = T.relu(T.matmul(xt, w1t.transpose(-2, -1)) + b1t)
        out = T.matmul(h, w2t.transpose(-2, -1))
        probe = np.linspace(-1.0, 1.0, int(np.prod(out.shape)), dtype=np.float32)
        loss = T.sum(out * T.tensor(probe.reshape(out.shape), backend=backend))
        loss.backward()
        # the bias gradient sums the relu gradient: find that node below it
        ops, n = [], b1t.grad.node
        for _ in range(6):
            ops.append(n.op)
            n = n.view_src if n.view_src is not None else (n.src[0] if n.src else None)
            if n is None:
                break
        want = T.OP["MATMUL_RELU_BACKWARD"] if fused else T.OP["RELU_BACKWARD"]
        assert want in ops, ops
        return out.numpy(), xt.grad.numpy(), w1t.grad.numpy(), b1t.grad.numpy(), w2t.grad.numpy()
    finally:
        T.FUSED_MATMUL_RELU_GRAD = prev


# (rows, in, hidden, out): the hidden layer's input-gradient product split or not
MLP2_SHAPES = [(64, 784, 128, 10), (128, 8192, 256, 100), (5, 7, 9, 3)]


# (rows, in, out): split-K folds (the epilogue in the fold) and unsplit products
LINEAR_SHAPES = [(64, 784, 128), (64, 128, 10), (128, 8192, 256), (128, 256, 100), (512, 64, 4096),
                 (3, 5, 7)]


# (shape, kernel, stride, padding): the 2x2 tiling kernel and the general one
POOL_GEOMETRIES = [((2, 3, 8, 8), 2, 2, 0), ((2, 3, 7, 9), 3, 2, 1), ((1, 2, 6, 6), 3, 1, 1)]


def pool_relu_input(shape, seed):
    """Uniform values with ties, NaN, signed zeros and negatives."""
    rng = np.random.default_rng(seed)
    x = rng.integers(-3, 4, shape).astype(np.float32) * np.float32(0.5)
    x.reshape(-1)[:4] = [np.nan, -0.0, 0.0, -1.0]
    return x


GRAPH_REWRITES = ("FOLD_CONSTANTS", "WEIGHT_GRAD_IN_PLACE_LAYOUT", "FUSED_ADD_RELU",
                  "FUSED_CONV_EPILOGUE", "FUSED_CONV_INPUT_GRAD", "FOLD_CONV_WEIGHT_GRAD",
                  "FUSED_POOL_RELU_GRAD", "FUSED_LINEAR_BIAS", "FUSED_MATMUL_RELU_GRAD",
                  "FUSED_CONV_POOL_GRAD", "FUSED_POOL_BIAS_GRAD")


def train_with_rewrites(backend, model_fn, batches, enabled, lr=0.1, momentum=0.9,
                        rewrites=GRAPH_REWRITES):
    """Losses and final parameters of SGD-momentum steps over `batches` with
    the tensor layer's graph rewrites in `rewrites` switched on or off."""
    from vkml_amd import nn, optim
    from vkml_amd import tensor as T

    saved = {r: getattr(T, r) for r in rewrites}
    try:
        for r in rewrites:
            setattr(T, r, enabled)
        model = model_fn(backend)
        opt = optim.SGD(model.parameters(), lr=lr, momentum=momentum)
        losses = []
        for x, y in batches:
            opt.zero_grad()
            loss = nn.cross_entropy(model(T.tensor(x, backend=backend)), T.tensor(y, backend=backend))
            loss.backward()
            opt.step()
            losses.append(np.float32(loss.item()))
        return np.array(losses), [p.numpy() for p in model.parameters()]
    finally:
        for r, v in saved.items():
            setattr(T, r, v)


def mlp_model(backend):
    """Config 1's MLP: Flatten, Linear(784,128), ReLU, Linear(128,10)."""
    from vkml_amd import nn

    nn.manual_seed(SEED)
    return nn.Sequential(nn.Flatten(), nn.Linear(784, 128, backend=backend), nn.ReLU(),
                         nn.Linear(128, 10, backend=backend))


def mlp_batches(steps, batch=64):
    rng = np.random.default_rng(SEED + 3)
    return [(rng.uniform(0, 1, (batch, 1, 28, 28)).astype(np.float32),
             rng.integers(0, 10, batch).astype(np.int64)) for _ in range(steps)]


def relu_inputs(shape, seed):
    """x and the output gradient g for the relu gradient, with NaN, +-0, +-inf
    in both (the select must pass NaN x through and keep g's bits)."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(shape).astype(np.float32)
    g = rng.standard_normal(shape).astype(np.float32)
    flat_x, flat_g = x.reshape(-1), g.reshape(-1)
    specials = np.array([np.nan, 0.0, -0.0, np.inf, -np.inf, 1e-45, -1e-45], np.float32)
    k = min(flat_x.size, specials.size)
    flat_x[:k] = specials[:k]
    flat_g[1:1 + k] = specials[:k][: max(0, min(k, flat_g.size - 1))]
    return x, g


def relu_grad(backend, x, g, fused):
    """d(relu(x))/dx applied to g on `backend`, as the RELU_BACKWARD node
    (fused=True) or as the reference's where/less_equal/zeros_like nodes."""
    from vkml_amd import tensor as T

    prev = T.FUSED_RELU_BACKWARD
    T.FUSED_RELU_BACKWARD = fused
    try:
        xt = T.tensor(x, requires_grad=True, backend=backend)
        T.backward(T.relu(xt), T.tensor(g, backend=backend))
        return xt.grad.numpy()
    finally:
        T.FUSED_RELU_BACKWARD = prev


def small_window(shape, cout, kernel, L):
    """Whether a weight gradient runs conv_wgrad_small_kernel: C*kh*kw <= 32,
    Cout <= 64, whole 32-position K-tiles per image and an image of at most
    8192 floats (staged in LDS)."""
    ck = shape[1] * kernel[0] * kernel[1]
    return ck <= 32 and cout <= 64 and L % 32 == 0 and shape[1] * shape[2] * shape[3] <= 8192


CONV_GEOMETRIES = [  # (x shape, Cout, kernel, stride, pad, dilation)
    ((2, 3, 5, 5), 4, (3, 3), (1, 1), (1, 1), (1, 1)),
    ((1, 2, 6, 6), 3, (2, 2), (2, 2), (0, 0), (1, 1)),
    ((2, 1, 7, 5), 2, (3, 2), (2, 1), (1, 0), (1, 1)),
    ((1, 2, 5, 5), 5, (2, 2), (1, 1), (0, 0), (2, 2)),
    ((3, 4, 9, 11), 6, (5, 3), (2, 3), (2, 1), (1, 2)),
    ((2, 3, 8, 8), 8, (1, 1), (1, 1), (0, 0), (1, 1)),
]


def ce_inputs(shape, seed):
    rng = np.random.default_rng(seed)
    logits = (rng.standard_normal(shape) * 3).astype(np.float32)
    labels = rng.integers(0, shape[1], shape[0]).astype(np.int64)
    labels[0] = shape[1] - 1
    if shape[0] > 2:
        labels[1] = shape[1]  # out of range: an all-zero one-hot row, as in the reference
    return logits, labels


# ---- the reference's known answers and fixtures (tests/golden) ----

_GOLDEN = None


def golden(name: str) -> dict:
    """One entry of tests/golden/reference_fixtures.json, lists as float32
    arrays (numbers stay numbers)."""
    global _GOLDEN
    if _GOLDEN is None:
        import json

        _GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_fixtures.json").read_text())

    def conv(v):
        if isinstance(v, list):
            return np.array(v, np.float32)
        if isinstance(v, dict):
            return {k: conv(x) for k, x in v.items()}
        return v

    return {k: conv(v) for k, v in _GOLDEN[name].items()}


# ---- BASELINE configs 1 and 5: the training streams (tests/golden/streams.py) ----

sys.path.insert(0, str(Path(__file__).parent / "golden"))
import streams  # noqa: E402

CONFIG5_STEPS = streams.CONFIG5.steps
CONFIG5_BATCH = streams.CONFIG5.batch
CONFIG5_LR = streams.CONFIG5.lr
CONFIG5_MOMENTUM = streams.CONFIG5.momentum
CONFIG5_LOSSES = streams.fixture_path(streams.CONFIG5)


def config5_model(backend):
    """conv(3->64,3x3)-ReLU-pool, conv(64->128,3x3)-ReLU-pool, flatten,
    Linear(8192,256)-ReLU, Linear(256,100), Kaiming-uniform from SEED."""
    return streams.model(streams.CONFIG5, backend)


def config5_batches(steps: int = CONFIG5_STEPS, batch: int = CONFIG5_BATCH):
    """A fresh batch per step, x ~ U[-1, 1) [batch, 3, 32, 32] and labels
    uniform in [0, 100), from one generator seeded SEED + batch."""
    return streams.batches(streams.CONFIG5, steps, batch)


def config5_train(backend, steps: int = CONFIG5_STEPS, batch: int = CONFIG5_BATCH) -> np.ndarray:
    """Per-step losses (float32) of config 5's SGD-momentum loop on `backend`."""
    return streams.train(streams.CONFIG5, backend, steps, batch)


def config5_golden_losses() -> np.ndarray:
    """The oracle's 100-step config-5 trajectory, written by
    tests/golden/make_training_losses.py (float32 bit patterns)."""
    return streams.oracle_losses(streams.CONFIG5)
