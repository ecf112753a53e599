"""The committed config-5 oracle trajectory (tests/golden/config5_cnn_losses.json)
against a live run of the CPU oracle: its first steps must be the same bits,
so the fixture the device test compares against is the oracle's, not a stale
copy. CPU only."""
from __future__ import annotations

import json

import numpy as np

from conftest import (CONFIG5_BATCH, CONFIG5_LOSSES, CONFIG5_LR, CONFIG5_MOMENTUM, CONFIG5_STEPS,
                      SEED, config5_golden_losses, config5_train)
from oracle import OracleBackend


def test_config5_fixture_describes_the_config():
    data = json.loads(CONFIG5_LOSSES.read_text())
    assert (data["seed"], data["model_seed"], data["batch"], data["steps"]) == \
        (SEED + CONFIG5_BATCH, SEED, CONFIG5_BATCH, CONFIG5_STEPS)
    assert (data["lr"], data["momentum"]) == (CONFIG5_LR, CONFIG5_MOMENTUM)
    losses = config5_golden_losses()
    assert losses.shape == (CONFIG5_STEPS,) and np.all(np.isfinite(losses))
    # the decimal copy is the same numbers
    assert np.array(data["losses"], np.float32).tobytes() == losses.tobytes()
    # cross-entropy over 100 classes starts near log(100)
    assert abs(float(losses[0]) - np.log(100.0)) < 0.1


def test_config5_fixture_matches_a_live_oracle_run():
    got = config5_train(OracleBackend(), steps=2)
    assert got.tobytes() == config5_golden_losses()[:2].tobytes()
