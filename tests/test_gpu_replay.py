"""Recorded programs (vkhip_program_*) and CapturedStep: a training step
recorded once and replayed, call by call or as one HIP graph, gives the same
bits as running the step eagerly, step after step (BASELINE configs 1 and 5).

Between replays the test runs eager work of its own and synchronises, and it
checks every replay against the eager trajectory, not only the last."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import SEED, config5_model
from vkml_amd import nn, optim
from vkml_amd import tensor as T

pytestmark = pytest.mark.gpu


def _mlp(backend):
    nn.manual_seed(SEED)
    return nn.Sequential(nn.Flatten(), nn.Linear(784, 128, backend=backend), nn.ReLU(),
                         nn.Linear(128, 10, backend=backend))


CONFIGS = {
    "mlp": (_mlp, (64, 1, 28, 28), (0.0, 1.0), 10, 0.1),
    "cnn": (config5_model, (128, 3, 32, 32), (-1.0, 1.0), 100, 0.01),
}


def _batches(config, steps):
    _, shape, (lo, hi), classes, _ = CONFIGS[config]
    rng = np.random.default_rng(SEED + 31)
    return [(rng.uniform(lo, hi, shape).astype(np.float32),
             rng.integers(0, classes, shape[0]).astype(np.int64)) for _ in range(steps)]


def _step_fn(model, opt):
    def fn(x, y):
        opt.zero_grad()
        loss = nn.cross_entropy(model(x), y)
        loss.backward()
        opt.step()
        return loss
    return fn


@pytest.mark.parametrize("graph", [False, True], ids=["replay", "graph"])
@pytest.mark.parametrize("config", ["mlp", "cnn"])
def test_replayed_steps_are_the_eager_steps_bit_for_bit(config, graph):
    dev = T.default_backend()
    make, _, _, _, lr = CONFIGS[config]
    batches = _batches(config, 8)

    model_e = make(dev)
    opt_e = optim.SGD(model_e.parameters(), lr=lr, momentum=0.9)
    fn_e = _step_fn(model_e, opt_e)
    eager = []
    for x, y in batches:
        eager.append(np.float32(fn_e(T.tensor(x, backend=dev), T.tensor(y, backend=dev)).item()))

    model_c = make(dev)
    opt_c = optim.SGD(model_c.parameters(), lr=lr, momentum=0.9)
    step = T.CapturedStep(_step_fn(model_c, opt_c), *batches[0], graph=graph)
    got = [np.float32(step.first[0])]
    probe = T.tensor(np.ones((256, 256), np.float32), backend=dev)
    for i, (x, y) in enumerate(batches[1:]):
        got.append(np.float32(step(x, y)[0]))
        # the program's own eager work and a synchronisation between replays
        s = T.sum(T.matmul(probe, probe)).item()
        assert s == 256.0 ** 3
        assert got[-1].tobytes() == eager[i + 1].tobytes(), f"replay {i + 1}"
    assert np.array(got).tobytes() == np.array(eager).tobytes()
    info = step.info()
    assert info["nodes"] > 0 and info["graph"] == graph
    for pe, pc in zip(model_e.parameters(), model_c.parameters()):
        assert pe.numpy().tobytes() == pc.numpy().tobytes()
    step.close()


@pytest.mark.parametrize("graph", [False, True], ids=["replay", "graph"])
@pytest.mark.parametrize("config", ["mlp", "cnn"])
def test_queued_steps_are_the_read_back_steps(config, graph):
    """Replays queued without reading the loss (read=False: the next step's
    uploads wait only for their staging slots) end in the same parameters and
    last loss as replays that read every loss back."""
    dev = T.default_backend()
    make, _, _, _, lr = CONFIGS[config]
    batches = _batches(config, 10)
    finals = []
    for queued in (False, True):
        model = make(dev)
        opt = optim.SGD(model.parameters(), lr=lr, momentum=0.9)
        step = T.CapturedStep(_step_fn(model, opt), *batches[0], graph=graph)
        last = None
        for x, y in batches[1:]:
            out = step(x, y, read=not queued)
            last = out[0] if out is not None else None
        if queued:
            assert last is None
            last = step.outputs_now()[0]
        finals.append((np.asarray(last).tobytes(), [p.numpy().tobytes() for p in model.parameters()]))
        step.close()
    assert finals[0] == finals[1]


@pytest.mark.parametrize("graph", [False, True], ids=["replay", "graph"])
@pytest.mark.parametrize("config", ["mlp", "cnn"])
def test_resident_inputs_and_device_loss_log_are_the_host_steps(config, graph):
    """Batches resident in HBM (DeviceArray inputs, copied on the device) and
    every step's loss kept in a device log (outputs_to, read once at the end,
    steps queued with read=False) give the losses and parameters of replays
    fed from host arrays that read every loss back."""
    from vkml_amd.device import DeviceArray

    dev = T.default_backend()
    make, _, _, _, lr = CONFIGS[config]
    batches = _batches(config, 8)
    runs = []
    for resident in (False, True):
        model = make(dev)
        opt = optim.SGD(model.parameters(), lr=lr, momentum=0.9)
        step = T.CapturedStep(_step_fn(model, opt), *batches[0], graph=graph)
        losses = [np.float32(step.first[0])]
        if resident:
            feed = [(DeviceArray.from_numpy(x), DeviceArray.from_numpy(y)) for x, y in batches]
            shape = step.outputs[0].shape
            log = DeviceArray((len(batches),) + tuple(shape), np.float32)
            for i in range(1, len(batches)):
                assert step(*feed[i], read=False) is None
                step.outputs_to(DeviceArray(shape, np.float32, None, log.buffer, offset=i))
            losses += list(log.numpy().reshape(len(batches))[1:])
        else:
            losses += [np.float32(step(x, y)[0]) for x, y in batches[1:]]
        runs.append((np.array(losses, np.float32).tobytes(),
                     [p.numpy().tobytes() for p in model.parameters()]))
        step.close()
    assert runs[0] == runs[1]


@pytest.mark.parametrize("graph", [False, True], ids=["replay", "graph"])
@pytest.mark.parametrize("config", ["mlp", "cnn"])
def test_prefetched_uploads_are_the_plain_uploads(config, graph):
    """Each call uploading the next batch on the copy stream (prefetch=) while
    its own step runs gives the losses and parameters of calls that upload
    their own batch: read back every step, queued (read=False), and with a
    prefetch the next call does not use (other array objects: they are
    uploaded instead), and from pinned host arrays (vkhip_host_alloc), which the
    DMA reads in place. The pageable host arrays are overwritten right after
    each prefetch: their bytes were copied when the call returned."""
    dev = T.default_backend()
    make, _, _, _, lr = CONFIGS[config]
    batches = _batches(config, 9)
    runs = []
    from vkml_amd.device import pinned_copy

    for variant in ("plain", "prefetch", "prefetch_queued", "prefetch_pinned"):
        model = make(dev)
        opt = optim.SGD(model.parameters(), lr=lr, momentum=0.9)
        step = T.CapturedStep(_step_fn(model, opt), *batches[0], graph=graph)
        losses = [np.float32(step.first[0])]
        if variant == "plain":
            losses += [np.float32(step(x, y)[0]) for x, y in batches[1:]]
        else:
            queued = variant == "prefetch_queued"
            pinned = variant == "prefetch_pinned"
            # pinned batches are read by the DMA in place (no scribbling there)
            feed = [(pinned_copy(x), pinned_copy(y)) if pinned else (x.copy(), y.copy()) for x, y in batches]
            step.prefetch(*feed[1])
            for i in range(1, len(feed)):
                x, y = feed[i]
                if i == 4:  # a fresh copy of the batch: the staged one is not used
                    x, y = batches[i][0].copy(), batches[i][1].copy()
                nxt = feed[i + 1] if i + 1 < len(feed) else None
                out = step(x, y, read=not queued, prefetch=nxt)
                if nxt is not None and not pinned:  # scribble over the host bytes just staged
                    nxt[0][...] = 7.0
                    nxt[1][...] = 0
                if queued:
                    assert out is None
                    losses.append(np.float32(step.outputs_now()[0]))
                else:
                    losses.append(np.float32(out[0]))
        runs.append((np.array(losses, np.float32).tobytes(),
                     [p.numpy().tobytes() for p in model.parameters()]))
        step.close()
    assert runs[1] == runs[0]
    assert runs[2] == runs[0]
    assert runs[3] == runs[0]


@pytest.mark.parametrize("config", ["mlp", "cnn"])
def test_early_outputs_are_the_step_end_outputs(config):
    """A plain replay's outputs read back early (vkhip_program_set_outputs: the
    units the loss depends on hoisted ahead of the backward pass and update,
    the bytes copied to pinned memory behind their last writer, the read
    waiting for that copy only) are the bytes the whole step leaves in the
    output tensor, and the reordering changes no unit's values: every loss
    and the final parameters equal those of replays read after the step ends,
    with the same node count. Graph replays declare no early outputs."""
    import ctypes

    from vkml_amd import _lib

    dev = T.default_backend()
    make, _, _, _, lr = CONFIGS[config]
    batches = _batches(config, 7)
    runs, infos = [], []
    for early in (False, True):
        model = make(dev)
        opt = optim.SGD(model.parameters(), lr=lr, momentum=0.9)
        step = T.CapturedStep(_step_fn(model, opt), *batches[0], early_outputs=early)
        losses = [np.float32(step.first[0])]
        for x, y in batches[1:]:
            out = step(x, y)
            if early:  # read before the step's end; the step's end leaves the same bytes
                assert out[0].tobytes() == step.outputs_now()[0].tobytes()
            losses.append(np.float32(out[0]))
        runs.append((np.array(losses, np.float32).tobytes(), [p.numpy().tobytes() for p in model.parameters()]))
        infos.append(step.info()["nodes"])
        step.close()
    assert runs[1] == runs[0]
    assert infos[1] == infos[0]
    model = make(dev)
    opt = optim.SGD(model.parameters(), lr=lr, momentum=0.9)
    step = T.CapturedStep(_step_fn(model, opt), *batches[0], graph=True)
    step(*batches[1])
    buf = np.empty(4, np.uint8)
    assert step.lib.vkhip_program_read_outputs(step._program, buf.ctypes.data_as(ctypes.c_void_p), 4) \
        == _lib.ERR_INVALID
    step.close()


def test_device_inputs_are_read_in_place_and_written_spans_refuse_binding():
    """A plain replay given DeviceArray inputs points its recorded inputs at
    them (vkhip_program_bind_input) instead of copying them in: the losses and
    parameters are those of host uploads, the recorded input tensors keep the
    recording's batch, a later host upload rebinds the recorded inputs, and a
    span a recorded call writes (the loss output) refuses a binding."""
    import ctypes

    from vkml_amd import _lib
    from vkml_amd.device import DeviceArray

    dev = T.default_backend()
    make, _, _, _, lr = CONFIGS["mlp"]
    batches = _batches("mlp", 6)
    runs = []
    for feed in ("host", "device"):
        model = make(dev)
        opt = optim.SGD(model.parameters(), lr=lr, momentum=0.9)
        step = T.CapturedStep(_step_fn(model, opt), *batches[0])
        losses = [np.float32(step.first[0])]
        for i, (x, y) in enumerate(batches[1:]):
            if feed == "device" and i != 2:  # call 3 uploads from the host between device calls
                x, y = DeviceArray.from_numpy(x), DeviceArray.from_numpy(y)
            losses.append(np.float32(step(x, y)[0]))
        if feed == "device":
            assert step.inputs[0].numpy().tobytes() == batches[3][0].tobytes()  # the last host upload
            out = step.outputs[0]
            ptr = out.node.storage.ptr + out.node.offset * out.node.itemsize
            assert step.lib.vkhip_program_bind_input(step._program, ctypes.c_void_p(ptr), ctypes.c_void_p(ptr),
                                                     4) == _lib.ERR_INVALID
        runs.append((np.array(losses, np.float32).tobytes(), [p.numpy().tobytes() for p in model.parameters()]))
        step.close()
    assert runs[1] == runs[0]


def test_constant_nodes_replay_only_while_nothing_else_writes_them():
    """A recorded constant (FULL) that no other recorded call writes keeps its
    recorded value and is left out of replays; one that another call
    overwrites (here a device copy into it) is recomputed every replay, so
    every replay sees the constant again."""
    dev = T.default_backend()
    x0 = np.arange(8, dtype=np.float32)

    def kept(x):
        return x + T.full((8,), 3.0, backend=dev)

    def overwritten(x):
        c = T.full((8,), 3.0, backend=dev)
        y = x + c
        T.realize([y])
        T.assign([c], [y])  # c's buffer now holds x + 3
        return y

    for fn in (kept, overwritten):
        step = T.CapturedStep(fn, x0)
        assert step.first[0].tobytes() == (x0 + 3).tobytes()
        for i in range(1, 4):
            x = x0 * i
            got = step(x)[0]
            assert got.tobytes() == (x + np.float32(3)).tobytes(), (fn.__name__, i)
        step.close()


def test_captured_step_checks_its_inputs():
    dev = T.default_backend()
    model = _mlp(dev)
    opt = optim.SGD(model.parameters(), lr=0.1)
    (x, y), = _batches("mlp", 1)
    step = T.CapturedStep(_step_fn(model, opt), x, y)
    with pytest.raises(ValueError):
        step(x[:32], y[:32])
    with pytest.raises(ValueError):
        step(x)
    from vkml_amd.device import DeviceArray
    with pytest.raises(ValueError):  # a device input of another shape
        step(DeviceArray.from_numpy(x[:32]), y)
    with pytest.raises(ValueError):  # a non-contiguous device input
        step(DeviceArray.from_numpy(np.ascontiguousarray(x.transpose(0, 1, 3, 2))).transpose(-2, -1), y)
    with pytest.raises(ValueError):  # a loss destination of the wrong size
        step.outputs_to(DeviceArray((2,), np.float32))
    with pytest.raises(ValueError):  # a prefetch of another shape
        step.prefetch(x[:32], y[:32])
    with pytest.raises(ValueError):  # prefetch takes host arrays
        step.prefetch(DeviceArray.from_numpy(x), y)
    step.close()
    with pytest.raises(RuntimeError):
        step(x, y)
