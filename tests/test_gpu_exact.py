"""The exact numerics mode (vkhip_set_numerics(VKHIP_NUMERICS_EXACT)): every
node the CPU oracle's bits. GEMMs and convolutions run on the exact arm
(rounded products, the oracle's pairwise order), softmax, log-softmax,
cross-entropy, exp and log use the oracle's exp/log methods and true division.
Whole training runs then follow the oracle step for step
(100 steps, compared live) and config 5 (100 steps at batch 128, against the
oracle's committed trajectory) meet the north star's 1e-4 loss-drift bar at
every step, bit for bit."""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from conftest import (CONFIG5_STEPS, CONV_GEOMETRIES, SEED, ce_inputs, ce_loss_and_grad,
                      config5_golden_losses, config5_train, conv_loss_and_grads,
                      conv_relu_loss_and_grads)
from oracle import OracleBackend
from vkml_amd import _lib, nn, ops, optim
from vkml_amd import tensor as T
from vkml_amd.device import DeviceArray

pytestmark = pytest.mark.gpu


@pytest.fixture
def exact(hip):
    hip.set_numerics("exact")
    assert hip.numerics() == "exact"
    try:
        yield T.default_backend()
    finally:
        hip.set_numerics("fast")


@pytest.fixture(scope="module")
def cpu():
    return OracleBackend()


def test_exact_exp_and_log_nodes(exact):
    rng = np.random.default_rng(SEED + 201)
    x = np.concatenate([np.linspace(-104, 89, 1_000_001, dtype=np.float32),
                        rng.uniform(-30, 5, 1_000_000).astype(np.float32),
                        np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45], np.float32)])
    got = T.exp(T.tensor(x, backend=exact)).numpy()
    assert got.tobytes() == O.expf(x).tobytes()
    y = np.concatenate([np.exp(np.linspace(-103, 88, 1_000_001)).astype(np.float32),
                        rng.uniform(1e-3, 1e3, 1_000_000).astype(np.float32),
                        np.array([0.0, -0.0, -1.0, np.inf, np.nan, 1e-45, 1.0], np.float32)])
    got = T.log(T.tensor(y, backend=exact)).numpy()
    assert got.tobytes() == O.logf(y).tobytes()


@pytest.mark.parametrize("shape,axis", [((4096, 1000), -1), ((64, 32768), -1), ((33, 300), 0),
                                        ((2, 3, 40, 5), 2), ((128, 100), -1), ((7, 1), -1)])
@pytest.mark.parametrize("log", [False, True])
def test_exact_softmax_is_the_oracle(exact, shape, axis, log):
    rng = np.random.default_rng(SEED + sum(shape) + axis)
    x = (rng.standard_normal(shape) * 2).astype(np.float32)
    fn = T.log_softmax if log else T.softmax
    got = fn(T.tensor(x, backend=exact), axis).numpy()
    want = O.softmax(x, axis, log=log)
    assert got.tobytes() == want.tobytes()


@pytest.mark.parametrize("shape", [(64, 10), (128, 100), (33, 300), (5, 2048)])
def test_exact_cross_entropy_is_the_oracle(exact, cpu, shape):
    logits, labels = ce_inputs(shape, shape[0] * 3 + shape[1])
    dl, dg = ce_loss_and_grad(exact, logits, labels, True)
    ol, og = ce_loss_and_grad(cpu, logits, labels, True)
    assert dl.tobytes() == ol.tobytes() and dg.tobytes() == og.tobytes()


@pytest.mark.parametrize("m,n,k,layout", [(64, 128, 784, "nt"), (128, 784, 64, "tn"),
                                          (256, 256, 4096, "nn"), (100, 37, 300, "tt")])
def test_exact_mode_routes_auto_gemms_to_the_exact_arm(exact, m, n, k, layout):
    rng = np.random.default_rng(SEED + m + n + k)
    a = rng.standard_normal((m, k), dtype=np.float32)
    b = rng.standard_normal((k, n), dtype=np.float32)
    da = DeviceArray.from_numpy(np.ascontiguousarray(a.T)).T if layout[0] == "t" else DeviceArray.from_numpy(a)
    db = DeviceArray.from_numpy(np.ascontiguousarray(b.T)).T if layout[1] == "t" else DeviceArray.from_numpy(b)
    assert ops.matmul(da, db).numpy().tobytes() == O.matmul(a, b).tobytes()
    # an explicit matrix-core request still runs the matrix cores
    mf = ops.matmul(da, db, kernel=_lib.GEMM_MFMA).numpy()
    assert np.max(np.abs(mf - O.matmul(a, b))) < 1e-3 * np.sqrt(k)


@pytest.mark.parametrize("shape,cout,kernel,stride,pad,dil",
                         CONV_GEOMETRIES + [((16, 64, 16, 16), 32, (3, 3), (1, 1), (1, 1), (1, 1))])
def test_exact_convolution_is_the_oracle(exact, cpu, shape, cout, kernel, stride, pad, dil):
    """CONV2D and CONV2D_WEIGHT_GRAD nodes on the exact arm (columns gathered
    from the image) and the rest of the conv graph (col2im of the dX product,
    bias sum): output and every gradient equal the oracle's im2col + matmul
    graph bit for bit."""
    rng = np.random.default_rng(SEED + 17)
    x = rng.uniform(-1, 1, shape).astype(np.float32)
    w = rng.uniform(-0.5, 0.5, (cout, shape[1]) + kernel).astype(np.float32)
    bias = rng.uniform(-0.5, 0.5, cout).astype(np.float32)
    dev = conv_loss_and_grads(exact, x, w, bias, stride, pad, dil, implicit=True)
    ref = conv_loss_and_grads(cpu, x, w, bias, stride, pad, dil, implicit=True)
    for got, want in zip(dev, ref):
        assert got.tobytes() == want.tobytes()


@pytest.mark.parametrize("shape,cout,kernel,stride,pad,dil",
                         CONV_GEOMETRIES + [((16, 64, 16, 16), 32, (3, 3), (1, 1), (1, 1), (1, 1))])
def test_exact_conv_bias_relu_is_the_oracle(exact, cpu, shape, cout, kernel, stride, pad, dil):
    """The CONV2D_BIAS_RELU node on the exact arm (bias and ReLU applied after
    the exact product) and its gradients: the oracle's bits."""
    rng = np.random.default_rng(SEED + 19)
    x = rng.uniform(-1, 1, shape).astype(np.float32)
    w = rng.uniform(-0.5, 0.5, (cout, shape[1]) + kernel).astype(np.float32)
    bias = rng.uniform(-0.5, 0.5, cout).astype(np.float32)
    dev = conv_relu_loss_and_grads(exact, x, w, bias, stride, pad, dil, True)
    ref = conv_relu_loss_and_grads(cpu, x, w, bias, stride, pad, dil, True)
    for got, want in zip(dev, ref):
        assert got.tobytes() == want.tobytes()


def _mlp(backend):
    nn.manual_seed(SEED)
    return nn.Sequential(nn.Flatten(), nn.Linear(784, 128, backend=backend), nn.ReLU(),
                         nn.Linear(128, 10, backend=backend))


@pytest.mark.timeout(300)
def test_config1_exact_100_steps_are_the_oracle(exact, cpu):
    rng = np.random.default_rng(SEED)
    batches = [(rng.uniform(0, 1, (64, 1, 28, 28)).astype(np.float32),
                rng.integers(0, 10, 64).astype(np.int64)) for _ in range(100)]
    res = {}
    for name, be in (("dev", exact), ("cpu", cpu)):
        model = _mlp(be)
        opt = optim.SGD(model.parameters(), lr=0.1, momentum=0.9)
        losses = []
        for x, y in batches:
            opt.zero_grad()
            loss = nn.cross_entropy(model(T.tensor(x, backend=be)), T.tensor(y, backend=be))
            loss.backward()
            opt.step()
            losses.append(np.float32(loss.item()))
        res[name] = (np.array(losses), [p.numpy() for p in model.parameters()])
    drift = np.abs(res["dev"][0].astype(np.float64) - res["cpu"][0])
    assert drift.max() <= 1e-4
    assert res["dev"][0].tobytes() == res["cpu"][0].tobytes()
    for a, b in zip(res["dev"][1], res["cpu"][1]):
        assert a.tobytes() == b.tobytes()


@pytest.mark.timeout(600)
def test_config5_exact_100_steps(exact):
    """BASELINE config 5 (CIFAR-100-shaped CNN, batch 128, SGD momentum 0.9)
    for 100 steps in the exact numerics mode against the oracle's trajectory
    (tests/golden/config5_cnn_losses.json): every step's loss within 1e-4 (the
    north star's bar), and in fact the same bits."""
    got = config5_train(exact)
    want = config5_golden_losses()
    drift = np.abs(got.astype(np.float64) - want.astype(np.float64))
    same = int(np.sum(got.view(np.uint32) == want.view(np.uint32)))
    print(f"config5 exact, 100 steps: max drift {drift.max():.3g} at step {drift.argmax()}, "
          f"{same}/{CONFIG5_STEPS} losses bit-identical", flush=True)
    assert drift.max() <= 1e-4, f"max loss drift {drift.max():.3g} at step {drift.argmax()}"
    assert same == CONFIG5_STEPS
