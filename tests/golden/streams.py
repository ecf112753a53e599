"""The seeded training streams of BASELINE configs 1 and 5, shared by the
parity tests, the scripts that write the oracle trajectories beside this file,
and bench.py's training entries, so that the loop a benchmark times is the loop
the parity tests check.

Config 1: Flatten -> Linear(784,128) -> ReLU -> Linear(128,10), batch 64,
x ~ U[0,1) [64,1,28,28], labels uniform in [0,10), SGD lr 0.1 momentum 0.9.
Config 5: conv(3->64)-ReLU-pool, conv(64->128)-ReLU-pool, flatten,
Linear(8192,256)-ReLU, Linear(256,100), batch 128, x ~ U[-1,1) [128,3,32,32],
labels uniform in [0,100), SGD lr 0.01 momentum 0.9.
Both: Kaiming-uniform weights from the model seed (reference python/vkml/nn.py
:31-44, 267-281, 680-691), a fresh batch per step from one numpy generator
(x first, then the labels), cross_entropy loss (reference src/api/ops.cpp
:417-441), 100 steps.
"""
from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent

# The reference suite's session seed (tests/python/test_vulkan_kernels.py:32).
SEED = 20260726


@dataclass(frozen=True)
class TrainingConfig:
    key: str            # fixture and bench entry name
    shape: tuple        # input batch shape
    classes: int
    lo: float           # x ~ U[lo, hi)
    hi: float
    lr: float
    momentum: float
    steps: int
    data_seed: int
    model_seed: int = SEED

    @property
    def batch(self) -> int:
        return self.shape[0]


CONFIG1 = TrainingConfig("mlp_784_128_10_b64", (64, 1, 28, 28), 10, 0.0, 1.0, 0.1, 0.9, 100,
                         data_seed=SEED)
CONFIG5 = TrainingConfig("cifar_cnn_b128", (128, 3, 32, 32), 100, -1.0, 1.0, 0.01, 0.9, 100,
                         data_seed=SEED + 128)
CONFIGS = {1: CONFIG1, 5: CONFIG5}


def batches(cfg: TrainingConfig, steps: int | None = None, batch: int | None = None):
    """The config's stream: one (x, labels) pair per step, generated lazily.
    A different batch size draws from the generator seeded for that size
    (config 5's live comparisons at small batches use this)."""
    batch = batch or cfg.batch
    seed = cfg.data_seed if batch == cfg.batch else cfg.data_seed - cfg.batch + batch
    rng = np.random.default_rng(seed)
    shape = (batch,) + tuple(cfg.shape[1:])
    for _ in range(cfg.steps if steps is None else steps):
        yield (rng.uniform(cfg.lo, cfg.hi, shape).astype(np.float32),
               rng.integers(0, cfg.classes, batch).astype(np.int64))


def model(cfg: TrainingConfig, backend=None):
    from vkml_amd import nn

    nn.manual_seed(cfg.model_seed)
    if cfg is CONFIG1:
        return nn.Sequential(nn.Flatten(), nn.Linear(784, 128, backend=backend), nn.ReLU(),
                             nn.Linear(128, 10, backend=backend))
    return nn.Sequential(
        nn.Conv2d(3, 64, 3, padding=1, backend=backend), nn.ReLU(), nn.MaxPool2d(2),
        nn.Conv2d(64, 128, 3, padding=1, backend=backend), nn.ReLU(), nn.MaxPool2d(2),
        nn.Flatten(), nn.Linear(8192, 256, backend=backend), nn.ReLU(),
        nn.Linear(256, 100, backend=backend))


def train(cfg: TrainingConfig, backend=None, steps: int | None = None,
          batch: int | None = None) -> np.ndarray:
    """Per-step losses (float32) of the config's SGD-momentum loop, every
    step's loss read back, on `backend` (None: the default device)."""
    from vkml_amd import nn, optim
    from vkml_amd import tensor as T

    net = model(cfg, backend)
    opt = optim.SGD(net.parameters(), lr=cfg.lr, momentum=cfg.momentum)
    losses = []
    for x, y in batches(cfg, steps, batch):
        opt.zero_grad()
        loss = nn.cross_entropy(net(T.tensor(x, backend=backend)), T.tensor(y, backend=backend))
        loss.backward()
        opt.step()
        losses.append(loss.item())
    return np.array(losses, np.float32)


def fixture_path(cfg: TrainingConfig, libm: bool = False) -> Path:
    stem = {CONFIG1.key: "config1_mlp_losses", CONFIG5.key: "config5_cnn_losses"}[cfg.key]
    return HERE / (stem + ("_libm" if libm else "") + ".json")


def fixture(cfg: TrainingConfig, libm: bool = False) -> dict:
    return json.loads(fixture_path(cfg, libm).read_text())


def oracle_losses(cfg: TrainingConfig, libm: bool = False) -> np.ndarray:
    """The committed CPU-oracle trajectory (float32 bit patterns): with the
    oracle's named exp/log methods, or with the platform libm's (libm=True)."""
    bits = np.array([int(h, 16) for h in fixture(cfg, libm)["losses_f32_bits"]], np.uint32)
    return bits.view(np.float32)


def max_drift(got: np.ndarray, want: np.ndarray) -> tuple[float, int]:
    """Largest |got - want| over the steps both cover (float64), and its step."""
    n = min(len(got), len(want))
    d = np.abs(np.asarray(got[:n], np.float64) - np.asarray(want[:n], np.float64))
    return float(d.max()), int(d.argmax())
