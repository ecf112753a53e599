"""Whole training steps on the device against the same graph on the CPU oracle.

BASELINE config 1 (MNIST-shaped MLP, 100 SGD-momentum steps) and config 5
(CIFAR-100-shaped CNN, batch 128, 100 steps) must keep every step's loss within
1e-4 of the oracle's (config 5 against the oracle's committed trajectory, plus
live comparisons of a few steps); config 4's conv layers are checked forward,
dX and dW at full shape. The graph, the initial weights and the data are identical on both
sides; only the backend executing the nodes differs.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import (CONV_GEOMETRIES, SEED, small_window, ce_inputs, ce_loss_and_grad,
                      config5_batches, config5_golden_losses, config5_model, config5_train, conv_loss_and_grads,
                      conv_relu_loss_and_grads, gemm_tolerance, mlp_batches, mlp_model, train_with_rewrites,
                      normwise_rel_err, relu_grad, relu_inputs, POOL_GEOMETRIES, pool_relu_input,
                      relu_pool_loss_and_grad, LINEAR_SHAPES, linear_loss_and_grads, MLP2_SHAPES,
                      mlp2_loss_and_grads, conv_pool_loss_and_grads, conv_pool_node, pool_bias_loss_and_grads)
from oracle import OracleBackend
from vkml_amd import nn, optim
from vkml_amd import tensor as T

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def backends():
    return T.default_backend(), OracleBackend()


def mlp(backend):
    nn.manual_seed(SEED)
    return nn.Sequential(nn.Flatten(), nn.Linear(784, 128, backend=backend), nn.ReLU(),
                         nn.Linear(128, 10, backend=backend))


def cnn(backend):
    nn.manual_seed(SEED)
    return nn.Sequential(
        nn.Conv2d(3, 64, 3, padding=1, backend=backend), nn.ReLU(), nn.MaxPool2d(2),
        nn.Conv2d(64, 128, 3, padding=1, backend=backend), nn.ReLU(), nn.MaxPool2d(2),
        nn.Flatten(), nn.Linear(8192, 256, backend=backend), nn.ReLU(),
        nn.Linear(256, 100, backend=backend))


def train(model, backend, batches, lr=0.1, momentum=0.9):
    opt = optim.SGD(model.parameters(), lr=lr, momentum=momentum)
    losses = []
    for x, y in batches:
        opt.zero_grad()
        loss = nn.cross_entropy(model(T.tensor(x, backend=backend)), T.tensor(y, backend=backend))
        loss.backward()
        opt.step()
        losses.append(loss.item())
    return np.array(losses)


@pytest.mark.timeout(600)
def test_config1_mlp_100_steps_loss_drift(backends):
    dev, cpu = backends
    rng = np.random.default_rng(SEED)
    batches = [(rng.uniform(0, 1, (64, 1, 28, 28)).astype(np.float32),
                rng.integers(0, 10, 64).astype(np.int64)) for _ in range(100)]
    got = train(mlp(dev), dev, batches)
    want = train(mlp(cpu), cpu, batches)
    drift = np.abs(got - want)
    assert drift.max() <= 1e-4, f"max loss drift {drift.max():.3g} at step {drift.argmax()}"
    assert got[-1] < got[0]


@pytest.mark.timeout(900)
@pytest.mark.parametrize("batch,steps", [(128, 2), (16, 10)])
def test_config5_cnn_loss_drift(backends, batch, steps):
    dev, cpu = backends
    rng = np.random.default_rng(SEED + batch)
    batches = [(rng.uniform(-1, 1, (batch, 3, 32, 32)).astype(np.float32),
                rng.integers(0, 100, batch).astype(np.int64)) for _ in range(steps)]
    got = train(cnn(dev), dev, batches, lr=0.01)
    want = train(cnn(cpu), cpu, batches, lr=0.01)
    drift = np.abs(got - want)
    assert drift.max() <= 1e-4, f"max loss drift {drift.max():.3g} at step {drift.argmax()}"


# How far the fast numerics may move config 5's 100-step trajectory, as a
# multiple of how far the reference's own CPU arithmetic moves it between two
# valid libm builds (the oracle with its named, correctly rounded exp/log
# against the oracle with glibc's expf/logf: tests/golden/config5_cnn_losses
# and config5_cnn_losses_libm). Both trajectories are the reference's CPU
# algorithm; the fast path differs from either by GEMM accumulation order
# (within 1e-5*sqrt(K) per product) and <= 2-ulp transcendentals.
FAST_PATH_ENVELOPE_FACTOR = 2.0


@pytest.mark.timeout(300)
def test_config5_cnn_fast_path_tracks_the_oracle(backends):
    """BASELINE config 5 at full batch (128), a fresh batch each step, all 100
    steps on the default (matrix-core) numerics against the CPU oracle's
    committed trajectory (tests/golden/config5_cnn_losses.json, written by
    tests/golden/make_training_losses.py and re-derived live for its first
    steps by tests/test_training_fixtures.py).

    The loop is chaotic at the rounding level (max-pool window choices and
    ReLU signs switch on last-bit differences): the oracle itself, with only
    its exp/log swapped for glibc's (1-ulp differences in ~1e-3 of the calls),
    agrees bit for bit for 11 steps, leaves 1e-4 at step 24 and is 1.8e-3
    off at step 86 (tests/test_training_fixtures.py pins these). So:
      - the first 15 steps stay within the north star's 1e-4;
      - all 100 stay within FAST_PATH_ENVELOPE_FACTOR times that
        oracle-against-oracle spread.
    The north star's 1e-4 for all 100 steps is met bit for bit by the exact
    numerics mode (test_config5_exact_numerics_100_steps)."""
    import streams as S

    dev, _ = backends
    got = config5_train(dev)
    want = config5_golden_losses()
    envelope, env_at = S.max_drift(want, S.oracle_losses(S.CONFIG5, libm=True))
    drift = np.abs(got.astype(np.float64) - want.astype(np.float64))
    print(f"config5 fast path, 100 steps: max drift {drift.max():.3g} at step {drift.argmax()}; "
          f"first 15 steps {drift[:15].max():.3g}; oracle named-vs-libm envelope {envelope:.3g} "
          f"(step {env_at}); ratio {drift.max() / envelope:.3g}", flush=True)
    assert drift[:15].max() <= 1e-4, f"max loss drift {drift[:15].max():.3g} at step {drift[:15].argmax()}"
    assert drift.max() <= FAST_PATH_ENVELOPE_FACTOR * envelope, \
        f"max loss drift {drift.max():.3g} at step {drift.argmax()} against envelope {envelope:.3g}"
    assert got[-1] < got[0] + 0.05  # training does not diverge


@pytest.mark.timeout(900)
@pytest.mark.parametrize("cin,cout", [(3, 64), (64, 128)])
def test_config4_conv_forward_dx_dw(backends, cin, cout):
    """Conv2d 3x3 s1 p1 on [128, cin, 32, 32]: output, dX (col2im of the TN
    product) and dW (NT product + batch reduce) against the oracle."""
    dev, cpu = backends
    rng = np.random.default_rng(SEED + cin)
    x = rng.uniform(-1, 1, (128, cin, 32, 32)).astype(np.float32)
    g = rng.standard_normal((128, cout, 32, 32)).astype(np.float32)
    res = {}
    for name, be in (("dev", dev), ("cpu", cpu)):
        nn.manual_seed(SEED)
        conv = nn.Conv2d(cin, cout, 3, padding=1, backend=be)
        xt = T.tensor(x, requires_grad=True, backend=be)
        y = conv(xt)
        y.backward(T.tensor(g, backend=be))
        res[name] = (y.numpy(), xt.grad.numpy(), conv.weight.grad.numpy(), conv.bias.grad.numpy())
    k = cin * 9
    assert normwise_rel_err(res["dev"][0], res["cpu"][0]) <= gemm_tolerance(k)
    assert normwise_rel_err(res["dev"][1], res["cpu"][1]) <= gemm_tolerance(cout)
    assert normwise_rel_err(res["dev"][2], res["cpu"][2]) <= gemm_tolerance(128 * 1024)
    # the bias gradient is a pure pairwise sum over axes {0, 2, 3}: bit-exact
    assert res["dev"][3].tobytes() == res["cpu"][3].tobytes()


@pytest.mark.parametrize("shape,cout,kernel,stride,pad,dil",
                         CONV_GEOMETRIES + [((128, 64, 16, 16), 128, (3, 3), (1, 1), (1, 1), (1, 1))])
def test_conv_node_on_device_is_bit_identical_to_the_graph(backends, shape, cout, kernel, stride,
                                                           pad, dil):
    """On the device, conv2d as one CONV2D node (implicit-im2col GEMM) gives
    the im2col + matmul graph's output and gradients bit for bit; against the
    oracle both are within the GEMM tolerance. With the weight gradient as one
    batch-summed node (the batch folded into the product's K axis when
    out_h*out_w is a multiple of 32) and the input gradient as one node (a
    convolution of the gradient for unit strides) the output and bias
    gradient keep those bits, dW is within the GEMM tolerance for
    K = N*out_h*out_w and dX for K = Cout*kh*kw."""
    dev, cpu = backends
    rng = np.random.default_rng(SEED + 7)
    x = rng.uniform(-1, 1, shape).astype(np.float32)
    w = rng.uniform(-0.5, 0.5, (cout, shape[1]) + kernel).astype(np.float32)
    bias = rng.uniform(-0.5, 0.5, cout).astype(np.float32)
    node = conv_loss_and_grads(dev, x, w, bias, stride, pad, dil, implicit=True, fold=False,
                               fused_dx=False)
    graph = conv_loss_and_grads(dev, x, w, bias, stride, pad, dil, implicit=False)
    positions = node[0][0, 0].size
    for i, (got, want) in enumerate(zip(node, graph)):
        if i == 2 and small_window(shape, cout, kernel, positions):
            # the small-window weight gradient sums in its own (fixed) order
            assert normwise_rel_err(got, want) <= gemm_tolerance(positions)
        else:
            assert got.tobytes() == want.tobytes()
    folded = conv_loss_and_grads(dev, x, w, bias, stride, pad, dil, implicit=True, fold=True,
                                 fused_dx=True)
    for i in (0, 3):
        assert folded[i].tobytes() == graph[i].tobytes()
    assert normwise_rel_err(folded[2], graph[2]) <= gemm_tolerance(shape[0] * positions)
    if positions % 32:
        assert folded[2].tobytes() == graph[2].tobytes()
    window = kernel[0] * kernel[1]
    assert normwise_rel_err(folded[1], graph[1]) <= gemm_tolerance(cout * window)
    if (stride != (1, 1) or any(d * (k - 1) < p for d, k, p in zip(dil, kernel, pad))
            or shape[1] < 32):
        assert folded[1].tobytes() == graph[1].tobytes()
    if shape[0] <= 4:
        ref = conv_loss_and_grads(cpu, x, w, bias, stride, pad, dil, implicit=True)
        ck = shape[1] * kernel[0] * kernel[1]
        for got, want, k in zip(node, ref, (ck, cout, shape[0] * node[0][0, 0].size, 1)):
            assert normwise_rel_err(got, want) <= gemm_tolerance(max(k, 2))


@pytest.mark.parametrize("shape,cout,kernel,stride,pad,dil",
                         CONV_GEOMETRIES + [((128, 64, 16, 16), 128, (3, 3), (1, 1), (1, 1), (1, 1)),
                                            ((128, 3, 32, 32), 64, (3, 3), (1, 1), (1, 1), (1, 1)),
                                            ((1, 64, 8, 8), 128, (3, 3), (1, 1), (1, 1), (1, 1))])
def test_conv_bias_relu_node_on_device_is_the_three_nodes(backends, shape, cout, kernel, stride, pad,
                                                          dil):
    """On the device, relu(conv2d(x, w, bias)) as one CONV2D_BIAS_RELU node
    (bias and ReLU in the conv kernel's epilogue, or in a pass after the
    split-K fold: the last geometry splits) gives the CONV2D + ADD + RELU
    graph's output and gradients bit for bit."""
    dev, cpu = backends
    rng = np.random.default_rng(SEED + 13)
    x = rng.uniform(-1, 1, shape).astype(np.float32)
    w = rng.uniform(-0.5, 0.5, (cout, shape[1]) + kernel).astype(np.float32)
    bias = rng.uniform(-0.5, 0.5, cout).astype(np.float32)
    print(f"conv_bias_relu x={shape} cout={cout} k={kernel}", flush=True)
    fused = conv_relu_loss_and_grads(dev, x, w, bias, stride, pad, dil, True)
    graph = conv_relu_loss_and_grads(dev, x, w, bias, stride, pad, dil, False)
    for got, want in zip(fused, graph):
        assert got.tobytes() == want.tobytes()


@pytest.mark.parametrize("rows,fan_in,hidden,fan_out", MLP2_SHAPES)
def test_matmul_relu_gradient_node_on_device(backends, rows, fan_in, hidden, fan_out):
    """On the device, the hidden relu's gradient as one MATMUL_RELU_BACKWARD
    node (the select in the split-K fold or a pass after an unsplit product)
    gives the device's MATMUL + RELU_BACKWARD graph bit for bit."""
    dev, _ = backends
    rng = np.random.default_rng(SEED + 18)
    x = rng.uniform(-1, 1, (rows, fan_in)).astype(np.float32)
    w1 = rng.uniform(-0.5, 0.5, (hidden, fan_in)).astype(np.float32)
    b1 = rng.uniform(-0.5, 0.5, hidden).astype(np.float32)
    w2 = rng.uniform(-0.5, 0.5, (fan_out, hidden)).astype(np.float32)
    print(f"matmul_relu_grad {rows}x{fan_in}->{hidden}->{fan_out}", flush=True)
    fused = mlp2_loss_and_grads(dev, x, w1, b1, w2, True)
    graph = mlp2_loss_and_grads(dev, x, w1, b1, w2, False)
    for got, want in zip(fused, graph):
        assert got.tobytes() == want.tobytes()


@pytest.mark.parametrize("relu", [False, True])
@pytest.mark.parametrize("rows,fan_in,fan_out", LINEAR_SHAPES)
def test_linear_bias_node_on_device(backends, rows, fan_in, fan_out, relu):
    """On the device, x @ w.T + bias (then relu) as one MATMUL_BIAS node (the
    epilogue in the split-K fold, or a pass after an unsplit product) gives the
    device's MATMUL + ADD (+ RELU) graph bit for bit."""
    dev, _ = backends
    rng = np.random.default_rng(SEED + 16)
    x = rng.uniform(-1, 1, (rows, fan_in)).astype(np.float32)
    w = rng.uniform(-0.5, 0.5, (fan_out, fan_in)).astype(np.float32)
    bias = rng.uniform(-0.5, 0.5, fan_out).astype(np.float32)
    print(f"linear_bias {rows}x{fan_in}->{fan_out} relu={relu}", flush=True)
    fused = linear_loss_and_grads(dev, x, w, bias, relu, True)
    graph = linear_loss_and_grads(dev, x, w, bias, relu, False)
    for got, want in zip(fused, graph):
        assert got.tobytes() == want.tobytes()


@pytest.mark.parametrize("shape,kernel,stride,pad",
                         POOL_GEOMETRIES + [((128, 64, 32, 32), 2, 2, 0), ((128, 128, 16, 16), 2, 2, 0)])
def test_pool_relu_gradient_node_on_device(backends, shape, kernel, stride, pad):
    """On the device, the relu gradient of max_pool2d(relu(x)) as one
    MAX_POOL2D_BACKWARD_RELU node gives the oracle's bits and the device's own
    two-node graph's, through the 2x2 tiling kernel and the general one."""
    dev, cpu = backends
    x = pool_relu_input(shape, SEED + 14)
    print(f"pool_relu x={shape} k={kernel} s={stride} p={pad}", flush=True)
    fused = relu_pool_loss_and_grad(dev, x, kernel, stride, pad, True)
    graph = relu_pool_loss_and_grad(dev, x, kernel, stride, pad, False)
    want = relu_pool_loss_and_grad(cpu, x, kernel, stride, pad, True)
    for got, two, ref in zip(fused, graph, want):
        assert got.tobytes() == two.tobytes()
        assert got.tobytes() == ref.tobytes()


# The CIFAR conv1 layer (the fused kernel), row widths 16 and 8 (fused, the
# fewest spans it takes), and two it leaves to the three nodes (width 12; a
# batch whose positions are no power of two).
CONV_POOL_DEVICE_LAYERS = [((128, 3, 32, 32), 64), ((4, 3, 16, 16), 16), ((8, 3, 8, 8), 32),
                           ((3, 4, 10, 12), 8), ((3, 3, 8, 8), 4)]


@pytest.mark.parametrize("shape,cout", CONV_POOL_DEVICE_LAYERS)
def test_conv_pool_gradient_node_on_device(backends, shape, cout):
    """On the device, the weight and bias gradients of
    max_pool2d(relu(conv2d(x, w, bias))) as one CONV2D_POOL_WEIGHT_BIAS_GRAD
    node give the bits of the device's own MAX_POOL2D_BACKWARD_RELU +
    CONV2D_WEIGHT_GRAD_SUM + SUM graph (pool windows with ties, pre-activations
    on 0). The node alone over the same x, y and pool gradient: the bias
    gradient is the oracle's bits (the pairwise tree's order), the weight
    gradient within the GEMM bar over K = N*oh*ow."""
    dev, cpu = backends
    rng = np.random.default_rng(SEED + 23)
    x = rng.integers(-1, 2, shape).astype(np.float32)
    w = (rng.integers(-1, 2, (cout, shape[1], 3, 3)) * 0.5).astype(np.float32)
    bias = (rng.integers(-1, 2, cout) * 0.5).astype(np.float32)
    print(f"conv_pool x={shape} cout={cout}", flush=True)
    fused = conv_pool_loss_and_grads(dev, x, w, bias, True)
    graph = conv_pool_loss_and_grads(dev, x, w, bias, False)
    for got, two in zip(fused, graph):
        assert got.tobytes() == two.tobytes()
    n_, c, h, w_ = shape
    xr = rng.uniform(-1, 1, shape).astype(np.float32)
    y = pool_relu_input((n_, cout, h, w_), SEED + 24)
    y = np.where(np.isnan(y), y, y + rng.uniform(0, 0.25, y.shape).astype(np.float32) * (y > 0))
    gp = rng.standard_normal((n_, cout, h // 2, w_ // 2)).astype(np.float32)
    got = conv_pool_node(dev, xr, y, gp, (3, 3), (1, 1))
    want = conv_pool_node(cpu, xr, y, gp, (3, 3), (1, 1))
    nw = cout * c * 9
    assert got[nw:].tobytes() == want[nw:].tobytes()
    assert normwise_rel_err(got[:nw], want[:nw]) <= gemm_tolerance(n_ * h * w_)


# CIFAR conv2's layer (the plane-sum kernel, rows of 16), rows of 32, and one
# it leaves to the pool backward and the reduction (rows of 10).
POOL_BIAS_DEVICE_LAYERS = [((128, 64, 16, 16), 128), ((4, 3, 32, 32), 8), ((3, 4, 6, 10), 5)]


@pytest.mark.parametrize("shape,cout", POOL_BIAS_DEVICE_LAYERS)
def test_pool_bias_gradient_node_on_device(backends, shape, cout):
    """On the device, a conv layer's bias gradient taken with its relu-masked
    pool gradient as one MAX_POOL2D_BACKWARD_RELU_BIAS node gives the device's
    own MAX_POOL2D_BACKWARD_RELU + SUM graph bit for bit (image, weight and
    bias gradients), and the node alone over the same pool gradient and layer
    output gives the oracle's bits, pool gradient and bias gradient both."""
    dev, cpu = backends
    rng = np.random.default_rng(SEED + 26)
    x = rng.integers(-1, 2, shape).astype(np.float32)
    w = (rng.integers(-1, 2, (cout, shape[1], 3, 3)) * 0.5).astype(np.float32)
    bias = (rng.integers(-1, 2, cout) * 0.5).astype(np.float32)
    print(f"pool_bias x={shape} cout={cout}", flush=True)
    fused = pool_bias_loss_and_grads(dev, x, w, bias, True)
    graph = pool_bias_loss_and_grads(dev, x, w, bias, False)
    for got, two in zip(fused, graph):
        assert got.tobytes() == two.tobytes()
    n_, _, h, w_ = shape
    y = pool_relu_input((n_, cout, h, w_), SEED + 27)
    gp = rng.standard_normal((n_, cout, h // 2, w_ // 2)).astype(np.float32)

    def node(backend):
        yt, gt = T.tensor(y, backend=backend), T.tensor(gp, backend=backend)
        out = T.Node(T.OP["MAX_POOL2D_BACKWARD_RELU_BIAS"], (y.size + cout,), np.float32, yt.node.backend,
                     [gt.node, yt.node], params=T._unfold_params((2, 2), (2, 2), (0, 0), (1, 1), (h, w_)))
        return T.Tensor(out).numpy()

    assert node(dev).tobytes() == node(cpu).tobytes()


@pytest.mark.parametrize("model", ["mlp", "cnn"])
def test_exact_graph_rewrites_keep_the_device_bits(backends, model):
    """On the device, the graph rewrites that compute the same arithmetic
    (constant folding, weight gradients in the weight's layout, fused
    add+relu, conv+bias+relu, pool+relu gradients, the conv layer's pool-fed
    weight and bias gradients and Linear bias epilogues) leave every loss and parameter of
    SGD-momentum training bit for bit unchanged: config 1's MLP for 10 steps,
    config 5's CNN at batch 128 for 3 steps."""
    dev, _ = backends
    rewrites = ("FOLD_CONSTANTS", "WEIGHT_GRAD_IN_PLACE_LAYOUT", "FUSED_ADD_RELU", "FUSED_CONV_EPILOGUE",
                "FUSED_POOL_RELU_GRAD", "FUSED_LINEAR_BIAS", "FUSED_MATMUL_RELU_GRAD", "FUSED_CONV_POOL_GRAD",
                "FUSED_POOL_BIAS_GRAD")
    if model == "mlp":
        fn, batches = mlp_model, mlp_batches(10)
    else:
        fn, batches = config5_model, list(config5_batches(3, 128))
    print(f"rewrites {model}", flush=True)
    on = train_with_rewrites(dev, fn, batches, True, rewrites=rewrites)
    off = train_with_rewrites(dev, fn, batches, False, rewrites=rewrites)
    assert on[0].tobytes() == off[0].tobytes()
    for a, b in zip(on[1], off[1]):
        assert a.tobytes() == b.tobytes()


@pytest.mark.parametrize("rows", [16384, 65536])
def test_weight_grad_layout_rewrite_keeps_bits_at_split_shapes(backends, rows):
    """A Linear(784, 128) weight gradient over 16384 and 65536 batch rows:
    the K-dominant products BASELINE config 3 names (128 x 784 x 16384). The
    device plans 128 x 784 and 784 x 128 over that K with different split-K
    partitions, so the in-place layout (g^T @ x) is not the reference
    layout's (x^T @ g)^T bits there; the host core must then keep the
    reference layout. The weight gradient is the same bytes with the rewrite
    on and off."""
    dev, _ = backends
    from vkml_amd import ops

    assert ops.gemm_plan(1, 128, 784, rows) != ops.gemm_plan(1, 784, 128, rows)
    rng = np.random.default_rng(SEED + rows)
    x = rng.standard_normal((rows, 784)).astype(np.float32)
    g = rng.standard_normal((rows, 128)).astype(np.float32)
    saved = T.WEIGHT_GRAD_IN_PLACE_LAYOUT
    grads = []
    try:
        for flag in (True, False):
            T.WEIGHT_GRAD_IN_PLACE_LAYOUT = flag
            nn.manual_seed(SEED)
            lin = nn.Linear(784, 128, bias=False, backend=dev)
            y = lin(T.tensor(x, backend=dev))
            y.backward(T.tensor(g, backend=dev))
            grads.append(lin.weight.grad.numpy())
    finally:
        T.WEIGHT_GRAD_IN_PLACE_LAYOUT = saved
    assert grads[0].tobytes() == grads[1].tobytes()
    # and both are the product within the GEMM bar (float64 check on rows)
    want = (g.astype(np.float64).T @ x.astype(np.float64))
    assert normwise_rel_err(grads[0], want) <= gemm_tolerance(rows)


def test_bias_gradient_reduce_is_bit_exact(backends):
    dev, cpu = backends
    x = np.random.default_rng(5).standard_normal((128, 64, 32, 32)).astype(np.float32)
    got = T.sum(T.tensor(x, backend=dev), [0, 2, 3]).numpy()
    want = T.sum(T.tensor(x, backend=cpu), [0, 2, 3]).numpy()
    assert got.tobytes() == want.tobytes()


@pytest.mark.parametrize("variant", [dict(momentum=0.9), dict(momentum=0.0),
                                     dict(momentum=0.9, weight_decay=1e-2, nesterov=True)])
def test_fused_sgd_on_device_is_bit_identical_to_the_oracle_graph(backends, variant):
    """The device's one-launch SGD step against the reference's ScaledAdd graph
    run by the CPU oracle: identical parameters, byte for byte, after 5 steps
    over parameters of the BASELINE MLP's shapes."""
    dev, cpu = backends
    rng = np.random.default_rng(SEED + 5)
    shapes = [(128, 784), (128,), (10, 128), (10,)]
    init = [rng.standard_normal(sh).astype(np.float32) for sh in shapes]
    grads = [[rng.standard_normal(sh).astype(np.float32) for sh in shapes] for _ in range(5)]

    def run(backend, fused):
        params = [T.tensor(w, requires_grad=True, backend=backend) for w in init]
        opt = optim.SGD(params, lr=0.1, fused=fused, **variant)
        for step in grads:
            for p, g in zip(params, step):
                p.grad = T.tensor(g, backend=backend)
            opt.step()
        return [p.numpy() for p in params]

    for a, b in zip(run(dev, True), run(cpu, False)):
        assert a.tobytes() == b.tobytes()


@pytest.mark.parametrize("shape", [(64, 10), (128, 100), (5, 37), (3, 2048), (7, 1), (33, 300),
                                   (4096, 1000)])
def test_fused_cross_entropy_on_device(backends, shape):
    """Device CROSS_ENTROPY nodes: byte for byte the device's own unfused graph
    (the log-softmax inside is the LOG_SOFTMAX kernel's arithmetic), and within
    tolerance of the oracle's."""
    dev, cpu = backends
    logits, labels = ce_inputs(shape, shape[0] * 7 + shape[1])
    fl, fg = ce_loss_and_grad(dev, logits, labels, True)
    ul, ug = ce_loss_and_grad(dev, logits, labels, False)
    assert fl.tobytes() == ul.tobytes() and fg.tobytes() == ug.tobytes()
    ol, og = ce_loss_and_grad(cpu, logits, labels, True)
    np.testing.assert_allclose(fl, ol, rtol=1e-5)
    assert normwise_rel_err(fg, og) <= gemm_tolerance(shape[1])


@pytest.mark.parametrize("shape", [(5, 7), (2, 3, 4, 5), (128, 64, 32, 32), (127, 3, 5), (1,)])
def test_fused_relu_backward_on_device(backends, shape):
    """Device RELU_BACKWARD: byte for byte the device's where/less_equal graph
    and the oracle's node (a select: exact), NaN/+-0/+-inf included; the
    vector path (contiguous, a multiple of 4) and the generic one both run."""
    dev, cpu = backends
    x, g = relu_inputs(shape, 29 + len(shape))
    fused = relu_grad(dev, x, g, True)
    assert fused.tobytes() == relu_grad(dev, x, g, False).tobytes()
    assert fused.tobytes() == relu_grad(cpu, x, g, True).tobytes()


@pytest.mark.parametrize("xs,ys", [((128, 64, 32, 32), (64, 1, 1)), ((128, 256), (256,)),
                                   ((4, 6, 8), (4, 1, 1)), ((2, 3, 4, 5), (3, 1, 1)),
                                   ((5, 12), (12,)), ((7, 3), (3,)), ((2, 3, 8), (2, 1, 8)),
                                   ((3, 4, 4), (1, 4, 1)), ((6, 10), (6, 1))])
def test_broadcast_binary_ops_on_device(backends, xs, ys):
    """add/sub/mul with a broadcast second operand (the bias adds: a value per
    channel over H*W runs, or a row of features repeated over the batch) take
    a vector path where the layout allows and the generic one elsewhere; every
    result is the oracle's, bit for bit."""
    dev, cpu = backends
    rng = np.random.default_rng(SEED + len(xs) * 10 + len(ys))
    x = rng.standard_normal(xs).astype(np.float32)
    y = rng.standard_normal(ys).astype(np.float32)
    for op in (T.add, T.sub, T.mul):
        got = op(T.tensor(x, backend=dev), T.tensor(y, backend=dev)).numpy()
        want = op(T.tensor(x, backend=cpu), T.tensor(y, backend=cpu)).numpy()
        assert got.tobytes() == want.tobytes(), op.__name__
