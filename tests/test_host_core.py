"""The host core (lazy graph, executor, autograd, nn, SGD) on the CPU oracle
backend, pinned against torch float64: forward values and every parameter
gradient of the BASELINE MLP and a small CNN, and SGD-with-momentum updates.
These check the restated graph (cross_entropy, conv2d lowering, autograd
rules) independently of the oracle's own kernels."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import (CONV_GEOMETRIES, SEED, ce_inputs, ce_loss_and_grad, conv_loss_and_grads,
                      config5_batches, config5_model, conv_relu_loss_and_grads, mlp_batches, mlp_model,
                      train_with_rewrites, POOL_GEOMETRIES, pool_relu_input, relu_pool_loss_and_grad,
                      LINEAR_SHAPES, linear_loss_and_grads, MLP2_SHAPES, mlp2_loss_and_grads,
                      relu_grad, relu_inputs, conv_pool_loss_and_grads)
from oracle import OracleBackend
from vkml_amd import nn, optim
from vkml_amd import tensor as T


@pytest.fixture(scope="module")
def cpu():
    return OracleBackend()


def torch_mlp_grads(x, y, w1, b1, w2, b2):
    p = [torch.tensor(v.astype(np.float64), requires_grad=True) for v in (w1, b1, w2, b2)]
    xt = torch.tensor(x.reshape(x.shape[0], -1).astype(np.float64))
    h = torch.relu(xt @ p[0].T + p[1])
    logits = h @ p[2].T + p[3]
    loss = torch.nn.functional.cross_entropy(logits, torch.tensor(y))
    loss.backward()
    return loss.item(), [q.grad.numpy() for q in p]


def test_mlp_forward_backward_vs_torch(cpu):
    rng = np.random.default_rng(SEED)
    x = rng.uniform(0, 1, (64, 1, 28, 28)).astype(np.float32)
    y = rng.integers(0, 10, 64).astype(np.int64)
    nn.manual_seed(SEED)
    model = nn.Sequential(nn.Flatten(), nn.Linear(784, 128, backend=cpu), nn.ReLU(),
                          nn.Linear(128, 10, backend=cpu))
    loss = nn.cross_entropy(model(T.tensor(x, backend=cpu)), T.tensor(y, backend=cpu))
    loss.backward()
    params = model.parameters()
    want_loss, want_grads = torch_mlp_grads(x, y, *[p.numpy() for p in params])
    assert abs(loss.item() - want_loss) <= 1e-5 * max(1.0, abs(want_loss))
    for p, g in zip(params, want_grads):
        got = p.grad.numpy()
        assert got.shape == g.shape
        np.testing.assert_allclose(got, g, rtol=1e-4, atol=1e-6)


def test_cnn_forward_backward_vs_torch(cpu):
    """conv -> relu -> pool -> flatten -> linear: conv2d lowered to
    im2col + batch-broadcast matmul, backward through col2im-free first conv,
    the NT weight-gradient GEMM + batch reduce, and max-pool backward."""
    rng = np.random.default_rng(SEED + 1)
    x = rng.uniform(-1, 1, (4, 3, 8, 8)).astype(np.float32)
    y = rng.integers(0, 5, 4).astype(np.int64)
    nn.manual_seed(SEED)
    conv = nn.Conv2d(3, 6, 3, padding=1, backend=cpu)
    conv2 = nn.Conv2d(6, 4, 3, padding=1, backend=cpu)
    fc = nn.Linear(4 * 2 * 2, 5, backend=cpu)
    model = nn.Sequential(conv, nn.ReLU(), nn.MaxPool2d(2), conv2, nn.ReLU(), nn.MaxPool2d(2),
                          nn.Flatten(), fc)
    loss = nn.cross_entropy(model(T.tensor(x, backend=cpu)), T.tensor(y, backend=cpu))
    loss.backward()
    tp = [torch.tensor(p.numpy().astype(np.float64), requires_grad=True)
          for p in model.parameters()]
    F = torch.nn.functional
    h = F.max_pool2d(F.relu(F.conv2d(torch.tensor(x, dtype=torch.float64), tp[0], tp[1], padding=1)), 2)
    h = F.max_pool2d(F.relu(F.conv2d(h, tp[2], tp[3], padding=1)), 2)
    logits = h.reshape(4, -1) @ tp[4].T + tp[5]
    want = F.cross_entropy(logits, torch.tensor(y))
    want.backward()
    assert abs(loss.item() - want.item()) <= 1e-5
    for p, q in zip(model.parameters(), tp):
        np.testing.assert_allclose(p.grad.numpy(), q.grad.numpy(), rtol=1e-4, atol=1e-6)


def test_sgd_momentum_matches_torch(cpu):
    rng = np.random.default_rng(3)
    w0 = rng.standard_normal((5, 3)).astype(np.float32)
    grads = [rng.standard_normal((5, 3)).astype(np.float32) for _ in range(3)]
    p = T.tensor(w0, requires_grad=True, backend=cpu)
    opt = optim.SGD([p], lr=0.1, momentum=0.9)
    tw = torch.tensor(w0, requires_grad=True)
    topt = torch.optim.SGD([tw], lr=0.1, momentum=0.9)
    for g in grads:
        p.grad = T.tensor(g, backend=cpu)
        opt.step()
        tw.grad = torch.tensor(g)
        topt.step()
        np.testing.assert_allclose(p.numpy(), tw.detach().numpy(), rtol=1e-6, atol=1e-7)


SGD_VARIANTS = [dict(momentum=0.0), dict(momentum=0.9), dict(momentum=0.9, weight_decay=1e-2),
                dict(momentum=0.9, nesterov=True), dict(momentum=0.5, weight_decay=0.1, nesterov=True),
                dict(momentum=0.0, weight_decay=1e-2)]


def sgd_run(cpu, fused_flags, variant, steps=4):
    rng = np.random.default_rng(11)
    shapes = [(7, 5), (5,), (3, 4, 2)]
    params = [T.tensor(rng.standard_normal(sh).astype(np.float32), requires_grad=True, backend=cpu)
              for sh in shapes]
    grads = [[rng.standard_normal(sh).astype(np.float32) for sh in shapes] for _ in range(steps)]
    opt = optim.SGD(params, lr=0.05, **variant)
    for k in range(steps):
        opt.fused = fused_flags[k % len(fused_flags)]
        for p, g in zip(params, grads[k]):
            p.grad = T.tensor(g, backend=cpu)
        opt.step()
    return [p.numpy() for p in params], grads


@pytest.mark.parametrize("variant", SGD_VARIANTS)
def test_fused_sgd_step_is_bit_identical_to_the_node_graph(cpu, variant):
    """One fused call per step against the reference's ScaledAdd graph, and a
    run that alternates between the two (the velocity carries over)."""
    nodes, _ = sgd_run(cpu, [False], variant)
    fused, _ = sgd_run(cpu, [True], variant)
    mixed, _ = sgd_run(cpu, [True, False], variant)
    for a, b, c in zip(nodes, fused, mixed):
        assert a.tobytes() == b.tobytes() == c.tobytes()


@pytest.mark.parametrize("variant", SGD_VARIANTS)
def test_sgd_variants_match_torch(cpu, variant):
    got, grads = sgd_run(cpu, [True], variant)
    rng = np.random.default_rng(11)
    shapes = [(7, 5), (5,), (3, 4, 2)]
    tp = [torch.tensor(rng.standard_normal(sh).astype(np.float32), requires_grad=True)
          for sh in shapes]
    topt = torch.optim.SGD(tp, lr=0.05, **variant)
    for k in range(len(grads)):
        for q, g in zip(tp, grads[k]):
            q.grad = torch.tensor(g)
        topt.step()
    for a, q in zip(got, tp):
        np.testing.assert_allclose(a, q.detach().numpy(), rtol=1e-6, atol=1e-7)


CE_SHAPES = [(64, 10), (128, 100), (5, 37), (3, 2048), (7, 1), (33, 300)]


@pytest.mark.parametrize("shape", CE_SHAPES)
def test_fused_cross_entropy_is_bit_identical_to_the_node_graph(cpu, shape):
    """The CROSS_ENTROPY / _BACKWARD nodes against the reference composition
    (log_softmax, one-hot, mul, sum, neg, mean and their autograd) on the
    oracle: same loss and same logits gradient, byte for byte."""
    logits, labels = ce_inputs(shape, shape[0] * 1000 + shape[1])
    fl, fg = ce_loss_and_grad(cpu, logits, labels, True)
    gl, gg = ce_loss_and_grad(cpu, logits, labels, False)
    assert fl.tobytes() == gl.tobytes() and fg.tobytes() == gg.tobytes()


@pytest.mark.parametrize("shape", [(5, 7), (2, 3, 4, 5), (128, 256), (1,)])
def test_fused_relu_backward_is_bit_identical_to_the_node_graph(cpu, shape):
    """The RELU_BACKWARD node against the reference's where(less_equal(x, 0),
    zeros, g) on the oracle, byte for byte, NaN/+-0/+-inf included; and the
    values torch's relu gradient gives on numbers (NaN x passes g through)."""
    x, g = relu_inputs(shape, 17 + len(shape))
    fused = relu_grad(cpu, x, g, True)
    graph = relu_grad(cpu, x, g, False)
    assert fused.tobytes() == graph.tobytes()
    want = np.where(x <= 0, np.float32(0.0), g)
    assert fused.tobytes() == want.astype(np.float32).tobytes()


@pytest.mark.parametrize("shape", [(64, 10), (128, 100)])
def test_fused_cross_entropy_matches_torch(cpu, shape):
    logits, labels = ce_inputs(shape, 5)
    labels[1] = 0  # torch rejects out-of-range labels
    loss, grad = ce_loss_and_grad(cpu, logits, labels, True)
    x = torch.tensor(logits.astype(np.float64), requires_grad=True)
    ref = torch.nn.functional.cross_entropy(x, torch.tensor(labels))
    ref.backward()
    np.testing.assert_allclose(loss, ref.item(), rtol=1e-6)
    np.testing.assert_allclose(grad, x.grad.numpy(), rtol=1e-5, atol=1e-7)


def test_views_and_broadcast_resolve_by_aliasing(cpu):
    a = np.arange(12, dtype=np.float32).reshape(3, 4)
    t = T.tensor(a, backend=cpu)
    np.testing.assert_array_equal(t.T.numpy(), a.T)
    np.testing.assert_array_equal((t + T.tensor(np.ones(4, np.float32), backend=cpu)).numpy(), a + 1)
    np.testing.assert_array_equal(T.sum(t, [0]).numpy(), a.sum(0))
    np.testing.assert_array_equal(T.matmul(t, t.T).numpy(), a @ a.T)


@pytest.mark.parametrize("model", ["mlp", "cnn"])
def test_graph_rewrites_keep_the_oracle_bits(cpu, model):
    """The tensor layer's graph rewrites (constant folding, weight gradients in
    place, fused add+relu and conv+bias+relu, the conv input-gradient and
    batch-folded weight-gradient nodes) leave every loss and parameter of
    SGD-momentum training on the oracle bit for bit unchanged: config 1's MLP
    for 4 steps, config 5's CNN at batch 4 for 2 steps."""
    if model == "mlp":
        fn, batches = mlp_model, mlp_batches(4)
    else:
        fn, batches = config5_model, list(config5_batches(2, 4))
    on = train_with_rewrites(cpu, fn, batches, True)
    off = train_with_rewrites(cpu, fn, batches, False)
    assert on[0].tobytes() == off[0].tobytes()
    for a, b in zip(on[1], off[1]):
        assert a.tobytes() == b.tobytes()


class _RecordingOracle(OracleBackend):
    """The oracle backend, noting the op of every node it is handed."""

    def __init__(self):
        super().__init__()
        self.ops = []
        self.flushes = 0

    def compute(self, nodes, count: int) -> None:
        self.ops.extend(int(nodes[i].op) for i in range(count))
        self.flushes += 1
        super().compute(nodes, count)


@pytest.mark.parametrize("model", ["mlp", "cnn"])
def test_reference_graph_hands_the_backend_reference_nodes_only(model):
    """Inside tensor.reference_graph() (and with SGD(fused=False)) a training
    step reaches the backend as the reference executor's node stream: every
    node a reference OpKind (ordinals below 96; the backend-extension nodes
    start there), im2col/col2im for convolutions, and the same losses and
    parameters, bit for bit, as the rewritten graph."""
    fn, batches = (mlp_model, mlp_batches(2)) if model == "mlp" else \
        (config5_model, list(config5_batches(2, 4)))
    res = {}
    for ref in (True, False):
        be = _RecordingOracle()
        net = fn(be)
        opt = optim.SGD(net.parameters(), lr=0.1, momentum=0.9, fused=not ref)
        losses = []
        for x, y in batches:
            ctx = T.reference_graph() if ref else None
            if ctx:
                ctx.__enter__()
            try:
                opt.zero_grad()
                loss = nn.cross_entropy(net(T.tensor(x, backend=be)), T.tensor(y, backend=be))
                loss.backward()
                opt.step()
                losses.append(np.float32(loss.item()))
            finally:
                if ctx:
                    ctx.__exit__(None, None, None)
        res[ref] = (np.array(losses), [p.numpy() for p in net.parameters()], be)
    ops_ref = set(res[True][2].ops)
    assert max(ops_ref) < 96, sorted(o for o in ops_ref if o >= 96)
    assert max(set(res[False][2].ops)) >= 96  # the rewritten graph does use extension nodes
    if model == "cnn":
        assert T.OP["IM2COL"] in ops_ref and T.OP["COL2IM"] in ops_ref
    # the switches are restored on exit
    assert T.IMPLICIT_CONV and T.FUSED_CROSS_ENTROPY and T.BACKWARD_FLUSH_EVERY > 0
    assert res[True][0].tobytes() == res[False][0].tobytes()
    for a, b in zip(res[True][1], res[False][1]):
        assert a.tobytes() == b.tobytes()


@pytest.mark.parametrize("rows,fan_in,hidden,fan_out", [MLP2_SHAPES[0], MLP2_SHAPES[-1]])
def test_matmul_relu_gradient_node_is_the_two_nodes(cpu, rows, fan_in, hidden, fan_out):
    """The hidden relu's gradient of relu(x @ w1.T + b1) @ w2.T as one
    MATMUL_RELU_BACKWARD node gives the MATMUL + RELU_BACKWARD graph's bits on
    the oracle (values, with negatives and zeros in the hidden layer)."""
    rng = np.random.default_rng(SEED + 17)
    x = rng.uniform(-1, 1, (rows, fan_in)).astype(np.float32)
    w1 = rng.uniform(-0.5, 0.5, (hidden, fan_in)).astype(np.float32)
    b1 = rng.uniform(-0.5, 0.5, hidden).astype(np.float32)
    w2 = rng.uniform(-0.5, 0.5, (fan_out, hidden)).astype(np.float32)
    fused = mlp2_loss_and_grads(cpu, x, w1, b1, w2, True)
    graph = mlp2_loss_and_grads(cpu, x, w1, b1, w2, False)
    for got, want in zip(fused, graph):
        assert got.tobytes() == want.tobytes()


@pytest.mark.parametrize("relu", [False, True])
@pytest.mark.parametrize("rows,fan_in,fan_out", LINEAR_SHAPES[:2] + LINEAR_SHAPES[-1:])
def test_linear_bias_node_is_the_three_nodes(cpu, rows, fan_in, fan_out, relu):
    """x @ w.T + bias (then relu) as one MATMUL_BIAS node gives the MATMUL +
    ADD (+ RELU) graph's output and gradients bit for bit on the oracle."""
    rng = np.random.default_rng(SEED + 15)
    x = rng.uniform(-1, 1, (rows, fan_in)).astype(np.float32)
    w = rng.uniform(-0.5, 0.5, (fan_out, fan_in)).astype(np.float32)
    bias = rng.uniform(-0.5, 0.5, fan_out).astype(np.float32)
    fused = linear_loss_and_grads(cpu, x, w, bias, relu, True)
    graph = linear_loss_and_grads(cpu, x, w, bias, relu, False)
    for got, want in zip(fused, graph):
        assert got.tobytes() == want.tobytes()


@pytest.mark.parametrize("shape,kernel,stride,pad", POOL_GEOMETRIES)
def test_pool_relu_gradient_node_is_the_two_nodes(cpu, shape, kernel, stride, pad):
    """The relu gradient of max_pool2d(relu(x)) as one MAX_POOL2D_BACKWARD_RELU
    node gives the MAX_POOL2D_BACKWARD + RELU_BACKWARD graph's bits on the
    oracle, with ties (first maximum), NaN, signed zeros and negatives."""
    x = pool_relu_input(shape, SEED + 12)
    fused = relu_pool_loss_and_grad(cpu, x, kernel, stride, pad, True)
    graph = relu_pool_loss_and_grad(cpu, x, kernel, stride, pad, False)
    for got, want in zip(fused, graph):
        assert got.tobytes() == want.tobytes()
    # and the mask is the relu's: x <= 0 gets +0 whatever the pool routed there
    g = fused[1]
    assert np.all(g[x <= 0] == 0) and not np.any(np.signbit(g[x <= 0]))


CONV_POOL_LAYERS = [((2, 3, 8, 8), 4), ((1, 2, 6, 10), 3), ((3, 1, 4, 4), 5)]


def conv_pool_operands(shape, cout, seed):
    """Small integers and halves: the conv outputs tie inside pool windows and
    sit exactly on the relu's 0."""
    rng = np.random.default_rng(seed)
    x = rng.integers(-1, 2, shape).astype(np.float32)
    w = (rng.integers(-1, 2, (cout, shape[1], 3, 3)) * 0.5).astype(np.float32)
    bias = (rng.integers(-1, 2, cout) * 0.5).astype(np.float32)
    return x, w, bias


@pytest.mark.parametrize("shape,cout", CONV_POOL_LAYERS)
def test_conv_pool_gradient_node_is_the_three_nodes(cpu, shape, cout):
    """The weight and bias gradients of max_pool2d(relu(conv2d(x, w, bias)))
    with x needing none, as one CONV2D_POOL_WEIGHT_BIAS_GRAD node, give the
    MAX_POOL2D_BACKWARD_RELU + CONV2D_WEIGHT_GRAD_SUM + SUM graph's bits on the
    oracle, with ties in the pool windows and pre-activations on 0."""
    x, w, bias = conv_pool_operands(shape, cout, SEED + 21)
    fused = conv_pool_loss_and_grads(cpu, x, w, bias, True)
    graph = conv_pool_loss_and_grads(cpu, x, w, bias, False)
    for got, want in zip(fused, graph):
        assert got.tobytes() == want.tobytes()
    assert np.any(bias != 0) and np.any(fused[2] != 0)


@pytest.mark.parametrize("shape,cout", [((2, 3, 16, 16), 4), ((1, 2, 6, 10), 3), ((2, 2, 32, 32), 2)])
def test_pool_bias_gradient_node_is_the_two_nodes(cpu, shape, cout):
    """A conv layer's bias gradient taken with its relu-masked pool gradient as
    one MAX_POOL2D_BACKWARD_RELU_BIAS node (the image needing its gradient)
    gives the MAX_POOL2D_BACKWARD_RELU + SUM graph's bits on the oracle, for
    the image, weight and bias gradients, with ties and pre-activations on 0."""
    from conftest import pool_bias_loss_and_grads

    x, w, bias = conv_pool_operands(shape, cout, SEED + 25)
    fused = pool_bias_loss_and_grads(cpu, x, w, bias, True)
    graph = pool_bias_loss_and_grads(cpu, x, w, bias, False)
    for got, want in zip(fused, graph):
        assert got.tobytes() == want.tobytes()
    assert np.any(fused[3] != 0)


def test_conv_pool_gradient_rewrite_needs_its_pattern(cpu):
    """No fused node when the image needs its gradient, or the pool is not 2x2
    at stride 2: the three nodes stay."""
    from vkml_amd import tensor as T

    x, w, bias = conv_pool_operands((2, 3, 8, 8), 4, SEED + 22)

    def weight_grad_source(x_grad, kernel, stride):
        xt = T.tensor(x, requires_grad=x_grad, backend=cpu)
        wt = T.tensor(w, requires_grad=True, backend=cpu)
        bt = T.tensor(bias, requires_grad=True, backend=cpu)
        out = T.max_pool2d(T.relu(T.conv2d(xt, wt, bt, 1, 1, 1)), kernel, stride)
        T.sum(out).backward()
        src = wt.grad.node
        while src.view_src is not None:
            src = src.view_src
        return src.op

    assert weight_grad_source(False, 2, 2) == T.OP["CONV2D_POOL_WEIGHT_BIAS_GRAD"]
    assert weight_grad_source(True, 2, 2) == T.OP["CONV2D_WEIGHT_GRAD_SUM"]
    assert weight_grad_source(False, 2, 1) == T.OP["CONV2D_WEIGHT_GRAD_SUM"]
    assert weight_grad_source(False, 3, 2) == T.OP["CONV2D_WEIGHT_GRAD_SUM"]


@pytest.mark.parametrize("shape,cout,kernel,stride,pad,dil", CONV_GEOMETRIES)
def test_conv_bias_relu_node_is_the_three_nodes(cpu, shape, cout, kernel, stride, pad, dil):
    """relu(conv2d(x, w, bias)) as one CONV2D_BIAS_RELU node gives the CONV2D +
    ADD + RELU graph's output and gradients bit for bit on the oracle (its
    relu gradient taken from the output), including NaN and signed-zero
    pre-activations."""
    rng = np.random.default_rng(SEED + 11)
    x = rng.uniform(-1, 1, shape).astype(np.float32)
    x.reshape(-1)[:3] = [np.nan, -0.0, 0.0]
    w = rng.uniform(-0.5, 0.5, (cout, shape[1]) + kernel).astype(np.float32)
    bias = rng.uniform(-0.5, 0.5, cout).astype(np.float32)
    fused = conv_relu_loss_and_grads(cpu, x, w, bias, stride, pad, dil, True)
    graph = conv_relu_loss_and_grads(cpu, x, w, bias, stride, pad, dil, False)
    for got, want in zip(fused, graph):
        assert got.tobytes() == want.tobytes()


@pytest.mark.parametrize("shape,cout,kernel,stride,pad,dil", CONV_GEOMETRIES)
def test_conv_node_matches_the_reference_graph(cpu, shape, cout, kernel, stride, pad, dil):
    """conv2d as one CONV2D node gives the reference graph's (im2col + matmul)
    output and x / weight / bias gradients bit for bit, with the weight
    gradient as per-image products + batch SUM or as one batch-summed node and
    the input gradient as TN product + col2im or as one node, and both agree with torch's float64 convolution."""
    rng = np.random.default_rng(SEED + 7)
    x = rng.uniform(-1, 1, shape).astype(np.float32)
    w = rng.uniform(-0.5, 0.5, (cout, shape[1]) + kernel).astype(np.float32)
    bias = rng.uniform(-0.5, 0.5, cout).astype(np.float32)
    node = conv_loss_and_grads(cpu, x, w, bias, stride, pad, dil, implicit=True, fold=False,
                               fused_dx=False)
    folded = conv_loss_and_grads(cpu, x, w, bias, stride, pad, dil, implicit=True, fold=True,
                                 fused_dx=True)
    graph = conv_loss_and_grads(cpu, x, w, bias, stride, pad, dil, implicit=False)
    for got, want in zip(node, graph):
        assert got.tobytes() == want.tobytes()
    # the batch-summed weight-gradient node is the per-image products and the
    # batch SUM on the oracle, the input-gradient node the TN product and
    # col2im: the same bits
    for got, want in zip(folded, graph):
        assert got.tobytes() == want.tobytes()
    xt = torch.tensor(x.astype(np.float64), requires_grad=True)
    wt = torch.tensor(w.astype(np.float64), requires_grad=True)
    bt = torch.tensor(bias.astype(np.float64), requires_grad=True)
    out = torch.nn.functional.conv2d(xt, wt, bt, stride, pad, dil)
    probe = torch.linspace(-1.0, 1.0, out.numel(), dtype=torch.float32).double().reshape(out.shape)
    (out * probe).sum().backward()
    np.testing.assert_allclose(node[0], out.detach().numpy(), rtol=1e-5, atol=1e-6)
    for got, want in zip(node[1:], (xt.grad, wt.grad, bt.grad)):
        np.testing.assert_allclose(got, want.numpy(), rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("every", [1, 3, 8])
def test_early_backward_flushes_give_the_same_training_steps(cpu, every):
    """Backward flushes the gradients built so far while it builds the rest
    (so the device starts on the forward pass early). The flushes only compute
    nodes the final one would, each once: three SGD steps of a small CNN give
    the same losses and parameters, bit for bit, as with one flush at the end,
    and the early flushes do happen."""
    rng = np.random.default_rng(SEED + 9)
    data = [(rng.uniform(-1, 1, (4, 3, 8, 8)).astype(np.float32),
             rng.integers(0, 5, 4).astype(np.int64)) for _ in range(3)]

    class Counting:
        def __init__(self, inner):
            self.inner, self.calls = inner, 0

        def __getattr__(self, name):
            return getattr(self.inner, name)

        def compute(self, nodes, count):
            self.calls += 1
            return self.inner.compute(nodes, count)

    def run(flush_every):
        be = Counting(cpu)
        prev = T.BACKWARD_FLUSH_EVERY, T.BACKWARD_FLUSH_MIN_BYTES
        T.BACKWARD_FLUSH_EVERY, T.BACKWARD_FLUSH_MIN_BYTES = flush_every, 0
        try:
            nn.manual_seed(SEED)
            model = nn.Sequential(nn.Conv2d(3, 6, 3, padding=1, backend=be), nn.ReLU(),
                                  nn.MaxPool2d(2), nn.Flatten(), nn.Linear(6 * 4 * 4, 5, backend=be))
            opt = optim.SGD(model.parameters(), lr=0.05, momentum=0.9)
            losses = []
            for x, y in data:
                opt.zero_grad()
                loss = nn.cross_entropy(model(T.tensor(x, backend=be)), T.tensor(y, backend=be))
                loss.backward()
                opt.step()
                losses.append(loss.numpy().tobytes())
            return losses, [p.numpy().tobytes() for p in model.parameters()], be.calls
        finally:
            T.BACKWARD_FLUSH_EVERY, T.BACKWARD_FLUSH_MIN_BYTES = prev

    want_losses, want_params, base_calls = run(0)
    losses, params, calls = run(every)
    assert losses == want_losses and params == want_params
    assert calls > base_calls


@pytest.mark.parametrize("fused", [True, False])
def test_pre_step_alias_sees_the_update_on_both_sgd_paths(cpu, fused):
    """assign() copies into the parameter's storage, as the reference's
    assign does (copy_device_to_device, python/vkml/__init__.py:153-165), and
    the fused step updates in place: a detach() taken before step() sees the
    new values on both paths, and both paths give the same bits."""
    rng = np.random.default_rng(SEED + 11)
    w = rng.standard_normal((6, 5)).astype(np.float32)
    g = rng.standard_normal((6, 5)).astype(np.float32)
    results = {}
    for path in (fused, not fused):
        p = T.tensor(w, requires_grad=True, backend=cpu)
        alias = p.detach()
        opt = optim.SGD([p], lr=0.1, momentum=0.9, fused=path)
        for _ in range(2):
            p.grad = T.tensor(g, backend=cpu)
            opt.step()
        results[path] = p.numpy()
        assert alias.numpy().tobytes() == results[path].tobytes()
        assert results[path].tobytes() != w.tobytes()
    assert results[True].tobytes() == results[False].tobytes()


def test_assign_checks_its_pairs(cpu):
    a = T.tensor(np.zeros((2, 3), np.float32), backend=cpu)
    with pytest.raises(ValueError):
        T.assign([a], [])
    with pytest.raises(ValueError):
        T.assign([a], [T.tensor(np.zeros((3, 2), np.float32), backend=cpu)])


@pytest.mark.parametrize("fused", ["FUSED_ADD_RELU", "FUSED_CONV_EPILOGUE"])
def test_fused_relu_nodes_follow_no_grad(cpu, fused):
    """relu() under no_grad on an ADD (or conv + bias ADD) built with grad
    enabled gives a node that does not require grad, as the unfused RELU
    does (the fused node takes requires_grad from the grad mode too)."""
    rng = np.random.default_rng(SEED + 31)
    w = T.tensor(rng.standard_normal((4, 3, 3, 3)).astype(np.float32), requires_grad=True, backend=cpu)
    b = T.tensor(rng.standard_normal(4).astype(np.float32), requires_grad=True, backend=cpu)
    x = T.tensor(rng.standard_normal((2, 3, 8, 8)).astype(np.float32), backend=cpu)
    if fused == "FUSED_ADD_RELU":
        pre = x.reshape(2, 192) + T.tensor(rng.standard_normal(192).astype(np.float32),
                                            requires_grad=True, backend=cpu)
    else:
        pre = T.conv2d(x, w, b, 1, 1)
    assert pre.requires_grad
    with T.no_grad():
        out = T.relu(pre)
    assert not out.requires_grad
    assert T.relu(pre).requires_grad
